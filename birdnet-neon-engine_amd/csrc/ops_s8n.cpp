// Registry kernels of the int8 path without dotprod (the reference's rt_ops_s8n.c contract: same op records, same
// validation, same outputs), run on the GPU for a batch of windows. Weights are repacked for the MFMA kernels once,
// at init, and kept in HBM.
#include <stdlib.h>
#include <string.h>

#include "bnh_internal.h"
#include "rt.h"

int bnh_proto_s8_init(rt_ctx *c, rt_op *op);  // ops_proto.cpp
int bnh_proto_s8_run(rt_ctx *c, rt_op *op);
void bnh_proto_s8_fini(rt_op *op);

// the int8 GEMM view of 4 tensors at ti (w, sw, colsum, b) and [N K Kp Np] at int params po (s8_view,
// src/rt_ops_s8n.c:13-25), uploaded as a bnh_s8w
static int s8_view(rt_ctx *c, rt_op *op, int ti, int po, bnh_s8w **out) {
  if (op->ni < po + 4) return rt_bad(c, op, "int8 GEMM shape [N K Kp Np] expected at int params %d..%d", po, po + 3);
  const int N = op->p[po], K = op->p[po + 1], Kp = op->p[po + 2], Np = op->p[po + 3];
  if (N <= 0 || K <= 0 || Np != ((N + 7) & ~7) || Kp != ((K + 15) & ~15))
    return rt_bad(c, op, "int8 GEMM shape N %d K %d Kp %d Np %d: expected Np = N rounded up to 8, Kp = K rounded up to 16",
                  N, K, Kp, Np);
  if (rt_need_t(c, op, ti, (size_t)Np * Kp, 0) || rt_need_t(c, op, ti + 1, (size_t)Np * 4, 1) ||
      rt_need_t(c, op, ti + 2, (size_t)Np * 4, 1) || rt_need_t(c, op, ti + 3, (size_t)Np * 4, 1))
    return RT_E_PARAM;
  *out = bnh_s8w_new(N, K, Kp, Np, (const int8_t *)rt_t(c, op, ti, nullptr), (const float *)rt_t(c, op, ti + 1, nullptr),
                     (const int32_t *)rt_t(c, op, ti + 2, nullptr), (const float *)rt_t(c, op, ti + 3, nullptr));
  if (!*out) return rt_oom(c, op, (size_t)Np * Kp);
  return 0;
}

// the output of a 1x1 conv (rt_pw_out_check, src/rt_ops_f32.c:183-196)
int rt_pw_out_check(rt_ctx *c, rt_op *op, int dt) {
  const int *p = op->p;
  int M = p[4], ldo = p[7], ow = p[8], opad = p[9];
  const rt_bufdesc *o = rt_bd(c, op, 1);
  if (!o) return rt_bad(c, op, "buffer argument 1 (output) is absent");
  if ((int)o->dtype != dt || o->ld != (uint32_t)ldo || o->halo != (uint32_t)opad)
    return rt_bad(c, op, "buffer argument 1 (buffer #%d, output): expected dtype %s ld %d halo %d, found dtype %s ld %u halo %u",
                  op->b[1], rt_dtype_name((uint32_t)dt), ldo, opad, rt_dtype_name(o->dtype), o->ld, o->halo);
  if (!opad) return rt_need(c, op, 1, dt, (size_t)M * ldo);
  RT_REQ(c, op, ow > 0 && M % ow == 0);
  if (o->W != (uint32_t)ow || (size_t)o->H * o->W != (size_t)M)
    return rt_bad(c, op, "buffer argument 1 (buffer #%d, padded output): expected %d x %d rows, found %u x %u", op->b[1],
                  M / ow, ow, o->H, o->W);
  return rt_need(c, op, 1, dt, (size_t)(M / ow + 2 * opad) * (ow + 2 * opad) * ldo);
}

typedef struct { bnh_s8w *W; } s8_state;
static void s8_fini(rt_op *op) {
  s8_state *s = (s8_state *)op->state;
  if (s) bnh_s8w_free(s->W);
  free(s);
}

// -------- PW_S8: b = [in f32 [M][lda], out, res | -1, q i8 [M4][Kp], sa f32 [M4], za i32 [M4] (, gate f32 [K] | -1)];
//          t = [w, sw, colsum, b]; p = [N K Kp Np, M, lda, act, ldo, ow, opad, ldr]   (src/rt_ops_s8n.c:92-134)
static int pw8_init(rt_ctx *c, rt_op *op) {
  s8_state *s = (s8_state *)calloc(1, sizeof *s);
  op->state = s;
  if (!s) return rt_oom(c, op, sizeof *s);
  if (rt_need_args(c, op, op->nb == 7 ? 7 : 6, 4, 11)) return RT_E_PARAM;
  const int *p = op->p;
  const int N = p[0], K = p[1], Kp = p[2], Np = p[3];
  if (N <= 0 || K <= 0 || Np != ((N + 7) & ~7) || Kp != ((K + 15) & ~15))
    return rt_bad(c, op, "int8 GEMM shape N %d K %d Kp %d Np %d: expected Np = N rounded up to 8, Kp = K rounded up to 16",
                  N, K, Kp, Np);
  if (op->nb == 7 && op->b[6] >= 0) {
    RT_REQ(c, op, K % 4 == 0 && K <= 4096);
    if (rt_need(c, op, 6, RT_F32, (size_t)K)) return RT_E_PARAM;
  }
  int M = p[4], lda = p[5], act = p[6], ldo = p[7], opad = p[9], ldr = p[10];
  size_t M4 = ((size_t)M + 3) & ~(size_t)3;
  RT_REQ(c, op, M > 0 && lda >= K && act >= 0 && act <= 2 && ldo >= Np && opad >= 0 && opad <= 3);
  const rt_bufdesc *r = rt_bd(c, op, 2);
  if (rt_need_nohalo(c, op, 0, RT_F32, (size_t)M * lda) || rt_pw_out_check(c, op, RT_F32)) return RT_E_PARAM;
  if (r) {
    RT_REQ(c, op, ldr >= Np && r->dtype == RT_F32 && r->ld == (uint32_t)ldr);
    if (r->halo) {
      RT_REQ(c, op, (size_t)r->H * r->W == (size_t)M && r->W > 0);
      if (rt_need(c, op, 2, RT_F32, (size_t)(r->H + 2 * r->halo) * (r->W + 2 * r->halo) * ldr)) return RT_E_PARAM;
    } else if (rt_need(c, op, 2, RT_F32, (size_t)M * ldr))
      return RT_E_PARAM;
  }
  if (rt_need(c, op, 3, RT_I8, M4 * Kp) || rt_need(c, op, 4, RT_F32, M4) || rt_need(c, op, 5, RT_I32, M4)) return RT_E_PARAM;
  return s8_view(c, op, 0, 0, &s->W);
}
static int pw8_run(rt_ctx *c, rt_op *op) {
  const s8_state *s = (const s8_state *)op->state;
  const int *p = op->p;
  const int B = c->nwin;
  if (op->quant_only)  // the depthwise op that reads the output recomputes the GEMM from the quantized rows
    return bnh_s8n_quant_rows((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[5], p[4], p[1], p[2], nullptr, 0,
                              (int8_t *)rt_b(c, op, 3), rt_ws(c, op, 3), (float *)rt_b(c, op, 4), rt_ws(c, op, 4),
                              (int32_t *)rt_b(c, op, 5), rt_ws(c, op, 5), B, c->stream);
  const rt_bufdesc *r = rt_bd(c, op, 2);
  const bool gated = op->nb == 7 && op->b[6] >= 0;
  bnh_epi32 e = {p[6], (float *)rt_b(c, op, 1), rt_ws(c, op, 1), p[7], p[8], p[9], (const float *)rt_b(c, op, 2),
                 rt_ws(c, op, 2), p[10], r ? (int)r->halo : 0, r ? (int)r->W : 0};
  if (!e.opad) e.ow = 0;
  if (e.opad && rt_halo_kept(c, op, 1)) {  // the halo is still zero from the arena: quantize and multiply only
    if (bnh_s8n_quant_rows((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[5], p[4], p[1], p[2],
                           gated ? (const float *)rt_b(c, op, 6) : nullptr, gated ? rt_ws(c, op, 6) : 0,
                           (int8_t *)rt_b(c, op, 3), rt_ws(c, op, 3), (float *)rt_b(c, op, 4), rt_ws(c, op, 4),
                           (int32_t *)rt_b(c, op, 5), rt_ws(c, op, 5), B, c->stream))
      return -1;
    return bnh_s8n_gemm((const int8_t *)rt_b(c, op, 3), rt_ws(c, op, 3), (const float *)rt_b(c, op, 4), rt_ws(c, op, 4),
                        (const int32_t *)rt_b(c, op, 5), rt_ws(c, op, 5), p[4], B, s->W, &e, c->stream);
  }
  return bnh_pw_s8((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[5], p[4],
                   gated ? (const float *)rt_b(c, op, 6) : nullptr, gated ? rt_ws(c, op, 6) : 0, (int8_t *)rt_b(c, op, 3),
                   rt_ws(c, op, 3), (float *)rt_b(c, op, 4), rt_ws(c, op, 4), (int32_t *)rt_b(c, op, 5), rt_ws(c, op, 5), B,
                   s->W, &e, c->stream);
}

// -------- GEMV_S8: b = [x f32 [K], out f32 [N], q i8 [4][Kp], sa f32 [4], za i32 [4]]; t = [w sw colsum b];
//          p = [N K Kp Np, act]   (src/rt_ops_s8n.c:136-158)
static int gemv8_init(rt_ctx *c, rt_op *op) {
  s8_state *s = (s8_state *)calloc(1, sizeof *s);
  op->state = s;
  if (!s) return rt_oom(c, op, sizeof *s);
  if (rt_need_args(c, op, 5, 4, 5)) return RT_E_PARAM;
  const int *p = op->p;
  const int N = p[0], K = p[1], Kp = p[2], Np = p[3];
  if (N <= 0 || K <= 0 || Np != ((N + 7) & ~7) || Kp != ((K + 15) & ~15))
    return rt_bad(c, op, "int8 GEMM shape N %d K %d Kp %d Np %d: expected Np = N rounded up to 8, Kp = K rounded up to 16",
                  N, K, Kp, Np);
  RT_REQ(c, op, p[4] == RT_ACT_NONE || p[4] == RT_ACT_RELU);
  if (rt_need(c, op, 0, RT_F32, (size_t)K) || rt_need(c, op, 1, RT_F32, (size_t)Np) ||
      rt_need(c, op, 2, RT_I8, (size_t)4 * Kp) || rt_need(c, op, 3, RT_F32, 4) || rt_need(c, op, 4, RT_I32, 4))
    return RT_E_PARAM;
  return s8_view(c, op, 0, 0, &s->W);
}
static int gemv8_run(rt_ctx *c, rt_op *op) {
  const s8_state *s = (const s8_state *)op->state;
  const int K = op->p[1], Np = op->p[3];
  bnh_epi32 e = {op->p[4], (float *)rt_b(c, op, 1), rt_ws(c, op, 1), Np, 0, 0, nullptr, 0, 0, 0, 0};
  return bnh_pw_s8((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), K, 1, nullptr, 0, (int8_t *)rt_b(c, op, 2),
                   rt_ws(c, op, 2), (float *)rt_b(c, op, 3), rt_ws(c, op, 3), (int32_t *)rt_b(c, op, 4), rt_ws(c, op, 4),
                   c->nwin, s->W, &e, c->stream);
}

static const rt_kernel K_PW_S8 = {pw8_init, pw8_run, s8_fini, "pw_s8n", 0x3a, 0x44};
static const rt_kernel K_GEMV_S8 = {gemv8_init, gemv8_run, s8_fini, "gemv_s8n", 0x1e, 0};
static const rt_kernel K_PROTO_S8 = {bnh_proto_s8_init, bnh_proto_s8_run, bnh_proto_s8_fini, "proto_s8n", 0xe, 0};

const bnh_s8w *rt_pw8_plain(const rt_op *op) {
  if (op->k != &K_PW_S8 || !op->state) return nullptr;
  if ((op->nb == 7 && op->b[6] >= 0) || op->b[2] >= 0 || op->p[9] == 0) return nullptr;
  return ((const s8_state *)op->state)->W;
}

const rt_kernel *rt_k_s8n(int base) {
  switch (base) {
    case RT_OP_PW_S8: return &K_PW_S8;
    case RT_OP_GEMV_S8: return &K_GEMV_S8;
    case RT_OP_PROTO_S8: return &K_PROTO_S8;
    default: return nullptr;
  }
}
