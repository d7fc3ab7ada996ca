// Registry kernels with fp16 arithmetic (variant 1, the reference's rt_ops_f16.c family) on the GPU.
#include "bnh_internal.h"
#include "rt.h"

int rt_dwk_check(rt_ctx *c, rt_op *op, size_t esz);             // ops_f32.cpp
int rt_dw3_check(rt_ctx *c, rt_op *op, int dt, int pt, int pl);  // ops_f32.cpp
int rt_dev_tensors(rt_ctx *c, rt_op *op, int n);
void rt_dev_fini(rt_op *op);
static inline const uint16_t *dev_h(const rt_op *op, int i) { return *((uint16_t *const *)op->state + i); }

// -------- DWK f16: as the fp32 op, fp16 buffers and tensors (src/rt_ops_f16.c:192-203)
static int dwk_init(rt_ctx *c, rt_op *op) {
  if (rt_dwk_check(c, op, 2)) return RT_E_PARAM;
  return rt_dev_tensors(c, op, 2);
}
static int dwk_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  return bnh_dwk_f16((const uint16_t *)rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], p[2], p[3], p[4], p[5], p[6],
                     dev_h(op, 0), dev_h(op, 1), p[9], (uint16_t *)rt_b(c, op, 1), rt_ws(c, op, 1), p[7], p[8],
                     (float *)rt_b(c, op, 2), rt_ws(c, op, 2), c->nwin, c->stream);
}

// -------- DW3 f16: b = [xp (halo 1), out, chsum f32]; t = [w f16 [9][C], b f16 [C]]; p = [H W C s Ho Wo pt pl]
//          (src/rt_ops_f16.c:83-122)
static int dw3_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 3, 2, 8)) return RT_E_PARAM;
  RT_REQ(c, op, op->p[2] <= 2048);
  if (rt_dw3_check(c, op, RT_F16, op->p[6], op->p[7])) return RT_E_PARAM;
  return rt_dev_tensors(c, op, 2);
}
static int dw3_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  return bnh_dw3_f16((const uint16_t *)rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], p[2], p[3], p[6], p[7],
                     dev_h(op, 0), dev_h(op, 1), (uint16_t *)rt_b(c, op, 1), rt_ws(c, op, 1), p[4], p[5],
                     (float *)rt_b(c, op, 2), rt_ws(c, op, 2), c->nwin, c->stream);
}

static const rt_kernel K_DW3 = {dw3_init, dw3_run, rt_dev_fini, "dw3_f16", 0x6, 0};
static const rt_kernel K_DWK = {dwk_init, dwk_run, rt_dev_fini, "dwk_f16", 0x6, 0};

const rt_kernel *rt_k_f16(int base) {
  switch (base) {
    case RT_OP_DW3: return &K_DW3;
    case RT_OP_DWK: return &K_DWK;
    default: return nullptr;
  }
}
