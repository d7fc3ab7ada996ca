// Registry kernels with fp32 arithmetic (variant 0 of the reference's rt_ops_f32.c family) on the GPU, plus the
// depthwise contract checks the fp16 family shares (as src/rt_ops_f32.c shares them with src/rt_ops_f16.c).
#include <stdlib.h>
#include <string.h>

#include "bnh_internal.h"
#include "rt.h"

// device copies of an op's first `n` tensors (weights / biases), freed by dev_fini
typedef struct { void *t[4]; } dev_state;
int rt_dev_tensors(rt_ctx *c, rt_op *op, int n) {
  dev_state *s = (dev_state *)calloc(1, sizeof *s);
  op->state = s;
  if (!s) return rt_oom(c, op, sizeof *s);
  for (int i = 0; i < n && i < 4; i++) {
    size_t nb = 0;
    const void *h = rt_t(c, op, i, &nb);
    s->t[i] = bnh_malloc(nb ? nb : 4);
    if (!s->t[i]) return rt_oom(c, op, nb);
    if (bnh_memcpy_h2d(s->t[i], h, nb)) return rt_bad(c, op, "uploading tensor argument %d: %s", i, bnh_last_error());
  }
  return 0;
}
void rt_dev_fini(rt_op *op) {
  dev_state *s = (dev_state *)op->state;
  if (s)
    for (int i = 0; i < 4; i++)
      if (s->t[i]) bnh_free(s->t[i]);
  free(s);
}
static inline void *dev_tn(const rt_op *op, int i) { return ((dev_state *)op->state)->t[i]; }

// -------- DWK: b = [xp (halo (k-1)/2), out [Ho][Wo][C], chsum f32 [C]]; t = [w [k*k][C], b [C]];
//          p = [H W C k s pt pl Ho Wo act]   (rt_dwk_check, src/rt_ops_f32.c:435-458)
int rt_dwk_check(rt_ctx *c, rt_op *op, size_t esz) {
  if (rt_need_args(c, op, 3, 2, 10)) return RT_E_PARAM;
  const int *p = op->p;
  const int H = p[0], W = p[1], C = p[2], k = p[3], s = p[4], pt = p[5], pl = p[6], Ho = p[7], Wo = p[8];
  const int h = (k - 1) / 2;
  RT_REQ(c, op, H > 0 && W > 0 && Ho > 0 && Wo > 0 && C > 0);
  RT_REQ(c, op, C % 8 == 0);
  RT_REQ(c, op, k % 2 == 1 && k >= 1 && k <= 7);
  RT_REQ(c, op, s >= 1 && s <= 2);
  RT_REQ(c, op, pt >= 0 && pt <= h && pl >= 0 && pl <= h);
  RT_REQ(c, op, p[9] >= 0 && p[9] <= 1);
  if (rt_need_t(c, op, 0, (size_t)k * k * C * esz, 0) || rt_need_t(c, op, 1, (size_t)C * esz, 0)) return RT_E_PARAM;
  RT_REQ(c, op, (Ho - 1) * s - pt + k <= H + 2 * h - h);  // the last tap of the last output stays in the halo
  RT_REQ(c, op, (Wo - 1) * s - pl + k <= W + 2 * h - h);
  const int dt = esz == 2 ? RT_F16 : RT_F32;
  if (rt_need_haloed(c, op, 0, dt, H, W, C, h)) return RT_E_PARAM;
  return rt_need(c, op, 1, dt, (size_t)Ho * Wo * C) || rt_need(c, op, 2, RT_F32, (size_t)C) ? RT_E_PARAM : 0;
}

// -------- DW3: b = [xp (halo 1), out, chsum f32]; t = [w [9][C], b [C]]; p = [H W C s Ho Wo (pt pl)]
//          (rt_dw3_check, src/rt_ops_f32.c:216-232)
int rt_dw3_check(rt_ctx *c, rt_op *op, int dt, int pt, int pl) {
  const int *p = op->p;
  const int H = p[0], W = p[1], C = p[2], s = p[3], Ho = p[4], Wo = p[5];
  const size_t esz = dt == RT_F16 ? 2 : 4;
  RT_REQ(c, op, H > 0 && W > 0 && Ho > 0 && Wo > 0 && C > 0);
  RT_REQ(c, op, C % 8 == 0);
  RT_REQ(c, op, s == 1 || s == 2);
  RT_REQ(c, op, pt >= 0 && pt <= 1 && pl >= 0 && pl <= 1);
  if (rt_need_t(c, op, 0, (size_t)9 * C * esz, 0) || rt_need_t(c, op, 1, (size_t)C * esz, 0)) return RT_E_PARAM;
  RT_REQ(c, op, (Ho - 1) * s - pt + 1 + 3 <= H + 2);
  RT_REQ(c, op, (Wo - 1) * s - pl + 1 + 3 <= W + 2);
  if (rt_need_haloed(c, op, 0, dt, H, W, C, 1)) return RT_E_PARAM;
  return rt_need(c, op, 1, dt, (size_t)Ho * Wo * C) || rt_need(c, op, 2, RT_F32, (size_t)C) ? RT_E_PARAM : 0;
}

static int dwk_init(rt_ctx *c, rt_op *op) {
  if (rt_dwk_check(c, op, 4)) return RT_E_PARAM;
  return rt_dev_tensors(c, op, 2);
}
static int dwk_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  return bnh_dwk_f32((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], p[2], p[3], p[4], p[5], p[6],
                     (const float *)dev_tn(op, 0), (const float *)dev_tn(op, 1), p[9], (float *)rt_b(c, op, 1),
                     rt_ws(c, op, 1), p[7], p[8], (float *)rt_b(c, op, 2), rt_ws(c, op, 2), c->nwin, c->stream);
}

static int dw3_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 3, 2, 6) || rt_dw3_check(c, op, RT_F32, 1, 1)) return RT_E_PARAM;
  return rt_dev_tensors(c, op, 2);
}
static int dw3_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  return bnh_dw3_f32((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], p[2], p[3],
                     (const float *)dev_tn(op, 0), (const float *)dev_tn(op, 1), (float *)rt_b(c, op, 1),
                     rt_ws(c, op, 1), p[4], p[5], (float *)rt_b(c, op, 2), rt_ws(c, op, 2), c->nwin, c->stream);
}

static const rt_kernel K_DW3 = {dw3_init, dw3_run, rt_dev_fini, "dw3_f32", 0x6, 0};
static const rt_kernel K_DWK = {dwk_init, dwk_run, rt_dev_fini, "dwk_f32", 0x6, 0};

const rt_kernel *rt_k_f32(int base) {
  switch (base) {
    case RT_OP_DW3: return &K_DW3;
    case RT_OP_DWK: return &K_DWK;
    default: return nullptr;
  }
}
