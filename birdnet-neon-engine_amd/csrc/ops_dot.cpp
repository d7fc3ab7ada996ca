// Registry kernels of the reference's dotprod + fp16 family (variant 2, src/rt_ops_dot.c): the mixed-precision plan
// of dense-conv models (BirdNET v3.0). The op contracts (argument counts, parameter checks, buffer and tensor
// requirements, message texts) are the reference's; the arithmetic runs on this library's GPU kernels:
//   STEM3     3 x 3 stride-2 fp32 conv of a 3-channel image into 24 fp16 channels (bit-identical);
//   CONV3C24  fp16 Winograd F(2x2,3x3) 24 -> 24, SiLU, + its own input (k_wino_f16: fp16 MFMA with fp32
//             accumulation and epilogue; within the fp16 Winograd tolerance of the reference's fp16 chains);
//   UNPAD     haloed fp16 -> fp32 rows (exact);
//   WINO_S8   int8 Winograd with per-tile dynamic quantisation (bit-identical).
#include <stdlib.h>
#include <string.h>

#include "bnh_internal.h"
#include "rt.h"

namespace {

// tensor argument i: fp32 with exactly `elems` elements (need_f32_t, src/rt_ops_dot.c:38-44)
int need_f32_t(rt_ctx *c, rt_op *op, int i, size_t elems) {
  if (rt_need_t(c, op, i, elems * 4, 0)) return RT_E_PARAM;
  const rt_tensor *t = rt_tensor_at(c->pkg, op->t[i], nullptr);
  if (t->dtype != RT_F32) return rt_bad(c, op, "tensor argument %d: expected fp32, found %s", i, rt_dtype_name(t->dtype));
  return 0;
}

// -------- STEM3: b = [img f32 [H][W][3] (no halo, stride 3), out f16 (halo 1) [Ho][Wo][24]];
//          t = [w OHWI [24][3][3][3], b [24]]; p = [H W Ho Wo]   (stem3_init / stem3_run, src/rt_ops_dot.c:46-61)
int stem3_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 2, 2, 4)) return RT_E_PARAM;
  const int *p = op->p;
  RT_REQ(c, op, p[0] >= 4 && p[1] >= 4 && p[0] % 2 == 0 && p[1] % 2 == 0 && p[2] == p[0] / 2 && p[3] == p[1] / 2);
  if (rt_need_haloed(c, op, 0, RT_F32, p[0], p[1], 3, 0) || rt_need_haloed(c, op, 1, RT_F16, p[2], p[3], 24, 1))
    return RT_E_PARAM;
  if (need_f32_t(c, op, 0, 24 * 27) || need_f32_t(c, op, 1, 24)) return RT_E_PARAM;
  return rt_dev_tensors(c, op, 2);
}
int stem3_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  uint16_t *out = (uint16_t *)rt_b(c, op, 1);
  if (!rt_halo_kept(c, op, 1) && bnh_zero_halo(out, rt_ws(c, op, 1), p[2], p[3], 24, 1, 2, c->nwin, c->stream))
    return -1;
  const rt_dev_state *s = (const rt_dev_state *)op->state;
  return bnh_stem3_f16((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], (const float *)s->t[0],
                       (const float *)s->t[1], out, rt_ws(c, op, 1), c->nwin, c->stream);
}

// -------- CONV3C24: b = [x f16 (halo 1) [H][W][24], out likewise]; the input is also the residual;
//          t = [w OHWI [24][3][3][24], b [24]]; p = [H W]   (c24_init / c24_run, src/rt_ops_dot.c:63-100)
void c24_fini(rt_op *op) { bnh_wino16_free((bnh_wino16 *)op->state); }
int c24_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 2, 2, 2)) return RT_E_PARAM;
  const int *p = op->p;
  RT_REQ(c, op, p[0] >= 2 && p[1] >= 2 && p[0] % 2 == 0 && p[1] % 2 == 0);  // 2x2 output tiles
  if (rt_need_haloed(c, op, 0, RT_F16, p[0], p[1], 24, 1) || rt_need_haloed(c, op, 1, RT_F16, p[0], p[1], 24, 1))
    return RT_E_PARAM;
  if (need_f32_t(c, op, 0, 24 * 9 * 24) || need_f32_t(c, op, 1, 24)) return RT_E_PARAM;
  bnh_wino16 *P =
      bnh_wino16_new(24, 24, (const float *)rt_t(c, op, 0, nullptr), (const float *)rt_t(c, op, 1, nullptr));
  op->state = P;
  return P ? 0 : rt_oom(c, op, 16 * 24 * 32 * 2);
}
int c24_run(rt_ctx *c, rt_op *op) {
  const int H = op->p[0], W = op->p[1];
  const uint16_t *x = (const uint16_t *)rt_b(c, op, 0);
  // SiLU(conv + b) + x into the zero-haloed output (the kernel zeroes the halo)
  return bnh_wino_f16(x, rt_ws(c, op, 0), H, W, 24, (const bnh_wino16 *)op->state, 1, (uint16_t *)rt_b(c, op, 1),
                      rt_ws(c, op, 1), 24, 1, x, rt_ws(c, op, 0), 24, 1, c->nwin, c->stream);
}

// -------- UNPAD: b = [x f16 (halo 1) [H][W][C], out f32 [H*W][C]]; p = [H W C]   (src/rt_ops_dot.c:109-128)
int unpad_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 2, 0, 3)) return RT_E_PARAM;
  const int *p = op->p;
  RT_REQ(c, op, p[0] > 0 && p[1] > 0 && p[2] > 0 && (p[1] * p[2]) % 8 == 0);
  if (rt_need_haloed(c, op, 0, RT_F16, p[0], p[1], p[2], 1)) return RT_E_PARAM;
  return rt_need_rows(c, op, 1, RT_F32, (size_t)p[0] * p[1], p[2]);
}
int unpad_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  return bnh_unpad_f16((const uint16_t *)rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], p[2], (float *)rt_b(c, op, 1),
                       rt_ws(c, op, 1), c->nwin, c->stream);
}

// -------- WINO_S8: b = [x f32 [H*W][C], out f16 [H*W][K]]; t = [w OHWI [K][3][3][C], b [K]]; p = [H W C K]
//          (wino_init / wino_run, src/rt_ops_dot.c:130-170). The quantised tiles live in an op-private device
//          workspace grown with the arena's window capacity.
struct wino_st {
  bnh_w8w *P;
  void *work;
  size_t cap;
};
void wino_fini(rt_op *op) {
  wino_st *s = (wino_st *)op->state;
  if (s) {
    bnh_wino8_free(s->P);
    if (s->work) bnh_free(s->work);
  }
  free(s);
}
int wino_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 2, 2, 4)) return RT_E_PARAM;
  const int *p = op->p;
  const int H = p[0], W = p[1], C = p[2], K = p[3];
  RT_REQ(c, op, H > 0 && W > 0 && C > 0 && C % 8 == 0 && C <= 2048 && K > 0 && K % 16 == 0 && K <= 2048);
  if (rt_need_rows(c, op, 0, RT_F32, (size_t)H * W, C) || rt_need_rows(c, op, 1, RT_F16, (size_t)H * W, K))
    return RT_E_PARAM;
  if (need_f32_t(c, op, 0, (size_t)K * 9 * C) || need_f32_t(c, op, 1, (size_t)K)) return RT_E_PARAM;
  wino_st *s = (wino_st *)calloc(1, sizeof *s);
  op->state = s;
  if (!s) return rt_oom(c, op, sizeof *s);
  s->P = bnh_wino8_new(C, K, (const float *)rt_t(c, op, 0, nullptr), (const float *)rt_t(c, op, 1, nullptr));
  return s->P ? 0 : rt_oom(c, op, (size_t)16 * K * C);
}
int wino_run(rt_ctx *c, rt_op *op) {
  wino_st *s = (wino_st *)op->state;
  const int *p = op->p;
  const size_t need = bnh_wino8_work_bytes(p[0], p[1], p[2], c->bcap);
  if (s->cap < need) {
    if (s->work) bnh_free(s->work);
    s->cap = 0;
    if (!(s->work = bnh_malloc(need))) {
      rt_oom(c, op, need);
      return -1;
    }
    s->cap = need;
  }
  return bnh_wino_s8((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], s->P, (uint16_t *)rt_b(c, op, 1),
                     rt_ws(c, op, 1), c->nwin, s->work, bnh_wino8_work_bytes(p[0], p[1], p[2], c->nwin), c->stream);
}

const rt_kernel K_STEM3 = {stem3_init, stem3_run, rt_dev_fini, "stem3_f32to16", 0x2, 0};
const rt_kernel K_CONV3C24 = {c24_init, c24_run, c24_fini, "conv3c24_wino16", 0x2, 0};
const rt_kernel K_UNPAD = {unpad_init, unpad_run, nullptr, "unpad_f16to32", 0x2, 0};
const rt_kernel K_WINO_S8 = {wino_init, wino_run, wino_fini, "wino3_s8", 0x2, 0};

}  // namespace

const rt_kernel *rt_k_dot(int base) {
  switch (base) {
    case RT_OP_STEM3: return &K_STEM3;
    case RT_OP_CONV3C24: return &K_CONV3C24;
    case RT_OP_UNPAD: return &K_UNPAD;
    case RT_OP_WINO_S8: return &K_WINO_S8;
    default: return nullptr;
  }
}
