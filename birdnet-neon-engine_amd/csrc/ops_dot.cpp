// Registry kernels of the reference's dotprod + fp16 family (variant 2, src/rt_ops_dot.c): the mixed-precision plan
// of dense-conv models (BirdNET v3.0). The op contracts (argument counts, parameter checks, buffer and tensor
// requirements, message texts) are the reference's; the arithmetic runs on this library's GPU kernels:
//   STEM3     3 x 3 stride-2 fp32 conv of a 3-channel image into 24 fp16 channels (bit-identical);
//   CONV3C24  fp16 Winograd F(2x2,3x3) 24 -> 24, SiLU, + its own input (k_wino_f16: fp16 MFMA with fp32
//             accumulation and epilogue; within the fp16 Winograd tolerance of the reference's fp16 chains);
//   UNPAD     haloed fp16 -> fp32 rows (exact);
//   WINO_S8   int8 Winograd with per-tile dynamic quantisation (bit-identical);
//   QCONV3    3 x 3 stride 1 / 2 conv, per-tensor int8 input, int8 GEMM + SiLU into fp16 (bit-identical);
//   QPW       1 x 1 conv with per-row int8 inputs (fp32, or gated fp16), fp16 / fp32 out (bit-identical);
//   SE_GATE16 the SE gate with fp16-held weights (bit-identical);
//   GEM_A     the generalised mean (the final power within one unit in the last place of the C library's powf);
//   HEADS_S8  dense + the two SED heads on int8 GEMMs (bit-identical).
#include <stdlib.h>
#include <string.h>

#include "bnh_internal.h"
#include "rt.h"

int bnh_proto8_dot_init(rt_ctx *c, rt_op *op);  // ops_proto.cpp
int bnh_proto8_dot_run(rt_ctx *c, rt_op *op);
void bnh_proto8_dot_fini(rt_op *op);

namespace {

// the reference's activation names, so the parameter-check messages read as its own
enum { ACT_NONE = RT_ACT_NONE, ACT_SILU = RT_ACT_SILU, ACT_RELU = RT_ACT_RELU };

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
  // one 256-byte-aligned slot per window, so that the two sub-batches of a split batch (running concurrently on
  // two streams) use disjoint slots: this sub-batch's start at window w0
  const size_t per = (bnh_wino8_work_bytes(p[0], p[1], p[2], 1) + 255) / 256 * 256;
  const size_t need = per * (size_t)c->bcap;
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
                     rt_ws(c, op, 1), c->nwin, (char *)s->work + per * c->w0, per * c->nwin, c->stream);
}

// TF-same output size and low pad of a k-tap stride-s axis (tf_same, src/rt_ops_dot.c:32-36)
void tf_same(int in, int k, int s, int *out, int *pad_lo) {
  const int o = (in + s - 1) / s, tot = (o - 1) * s + k - in;
  *out = o;
  *pad_lo = tot < 0 ? 0 : tot / 2;
}

// -------- QCONV3: b = [x f32 [H*W][C], out f16 [Ho*Wo][K]]; t = [w OHWI [K][3][3][C], b [K]]; p = [H W C K s Ho Wo]
//          (qconv_init / qconv_run, src/rt_ops_dot.c:186-216): per-tensor int8 input in a zero-point-haloed copy
//          (op-private device scratch), the implicit-im2col int8 GEMM + SiLU into fp16 rows.
struct qc_st {
  bnh_qdw *q;
  int pt, pl;
  void *work;
  size_t cap, ws;
};
void qconv_fini(rt_op *op) {
  qc_st *s = (qc_st *)op->state;
  if (s) {
    bnh_qdw_free(s->q);
    if (s->work) bnh_free(s->work);
  }
  free(s);
}
int qconv_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 2, 2, 7)) return RT_E_PARAM;
  const int *p = op->p;
  int H = p[0], W = p[1], C = p[2], K = p[3], s = p[4], Ho, Wo, pt, pl;
  RT_REQ(c, op, H > 0 && W > 0 && C > 0 && C % 8 == 0 && K > 0 && K % 16 == 0 && (s == 1 || s == 2));
  tf_same(H, 3, s, &Ho, &pt);
  tf_same(W, 3, s, &Wo, &pl);
  RT_REQ(c, op, p[5] == Ho && p[6] == Wo); /* TF-same geometry */
  if (rt_need_rows(c, op, 0, RT_F32, (size_t)H * W, C) || rt_need_rows(c, op, 1, RT_F16, (size_t)Ho * Wo, K))
    return RT_E_PARAM;
  if (need_f32_t(c, op, 0, (size_t)K * 9 * C) || need_f32_t(c, op, 1, (size_t)K)) return RT_E_PARAM;
  qc_st *st = (qc_st *)calloc(1, sizeof *st);
  op->state = st;
  if (!st) return rt_oom(c, op, sizeof *st);
  st->pt = pt;
  st->pl = pl;
  st->ws = bnh_qconv3_work_bytes(H, W, C);
  st->q = bnh_qdw_new((const float *)rt_t(c, op, 0, nullptr), (const float *)rt_t(c, op, 1, nullptr), K, 9 * C, K);
  return st->q ? 0 : rt_oom(c, op, (size_t)K * 9 * C);
}
int qconv_run(rt_ctx *c, rt_op *op) {
  qc_st *st = (qc_st *)op->state;
  const int *p = op->p;
  const size_t need = st->ws * (size_t)c->bcap;
  if (st->cap < need) {
    if (st->work) bnh_free(st->work);
    st->cap = 0;
    if (!(st->work = bnh_malloc(need))) {
      rt_oom(c, op, need);
      return -1;
    }
    st->cap = need;
  }
  return bnh_qconv3((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], p[2], p[4], st->pt, st->pl, p[5],
                    p[6], st->q, (uint16_t *)rt_b(c, op, 1), rt_ws(c, op, 1), c->nwin,
                    (char *)st->work + st->ws * c->w0, st->ws, c->stream);  // this sub-batch's window slots
}

// -------- QPW: b = [in, out, a8 int8 [M][Kp], rq f32 [2 M], res f32 | -1, gate f16 [K] | -1]; t = [w [N][K], b [N]];
//          p = [N K M in_dt ldx act out_dt ldo ow opad]   (qpw_init / qpw_run, src/rt_ops_dot.c:231-339)
// in_dt RT_F32: fp32 rows; RT_F16: fp16 rows, each channel first multiplied by the gate (an SE) when one is given.
// out_dt RT_F16: fp16, zero-haloed by opad (ow = the image width) when opad > 0; RT_F32: fp32 rows + residual.
void qw_fini(rt_op *op) { bnh_qdw_free((bnh_qdw *)op->state); }
int qpw_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 6, 2, 10)) return RT_E_PARAM;
  const int *p = op->p;
  int N = p[0], K = p[1], M = p[2], idt = p[3], ldx = p[4], act = p[5], odt = p[6], ldo = p[7], ow = p[8], opad = p[9];
  int Kp = (K + 15) & ~15;
  RT_REQ(c, op, N > 0 && N % 16 == 0 && K > 0 && K % 8 == 0 && M > 0 && ldx >= K && ldo >= N);
  RT_REQ(c, op, (idt == RT_F32 || idt == RT_F16) && (odt == RT_F32 || odt == RT_F16));
  RT_REQ(c, op, act == ACT_NONE || act == ACT_SILU || (act == ACT_RELU && odt == RT_F32));
  RT_REQ(c, op, opad == 0 || (opad == 1 && odt == RT_F16 && ow > 0 && M % ow == 0 && ldo == N));
  RT_REQ(c, op, op->b[4] < 0 || (odt == RT_F32 && opad == 0)); /* residual: fp32 rows */
  RT_REQ(c, op, op->b[5] < 0 || idt == RT_F16);                /* gate: fp16 input */
  if (rt_need_nohalo(c, op, 0, idt, (size_t)M * ldx)) return RT_E_PARAM;
  if (opad) {
    if (rt_need_haloed(c, op, 1, RT_F16, M / ow, ow, ldo, 1)) return RT_E_PARAM;
  } else if (rt_need_rows(c, op, 1, odt, (size_t)M, ldo))
    return RT_E_PARAM;
  if (rt_need(c, op, 2, RT_I8, (size_t)(M + 4) * Kp) || rt_need(c, op, 3, RT_F32, (size_t)2 * (M + 4)))
    return RT_E_PARAM;
  if (op->b[4] >= 0 && rt_need(c, op, 4, RT_F32, (size_t)M * ldo)) return RT_E_PARAM;
  if (op->b[5] >= 0 && rt_need(c, op, 5, RT_F16, (size_t)K)) return RT_E_PARAM;
  if (need_f32_t(c, op, 0, (size_t)N * K) || need_f32_t(c, op, 1, (size_t)N)) return RT_E_PARAM;
  bnh_qdw *q = bnh_qdw_new((const float *)rt_t(c, op, 0, nullptr), (const float *)rt_t(c, op, 1, nullptr), N, K, N);
  op->state = q;
  return q ? 0 : rt_oom(c, op, (size_t)N * Kp);
}
int qpw_run(rt_ctx *c, rt_op *op) {
  const bnh_qdw *q = (const bnh_qdw *)op->state;
  const int *p = op->p;
  const int N = p[0], K = p[1], M = p[2], Kp = (K + 15) & ~15;
  int8_t *a8 = (int8_t *)rt_b(c, op, 2);
  float *rq = (float *)rt_b(c, op, 3);
  if (bnh_qd_quant_rows(rt_b(c, op, 0), p[3] == RT_F16, rt_ws(c, op, 0), p[4], M, K, (const uint16_t *)rt_b(c, op, 5),
                        rt_ws(c, op, 5), a8, rt_ws(c, op, 2), rq, rt_ws(c, op, 3), c->nwin, c->stream))
    return -1;
  void *out = rt_b(c, op, 1);
  if (p[9] && !rt_halo_kept(c, op, 1) &&
      bnh_zero_halo(out, rt_ws(c, op, 1), M / p[8], p[8], p[7], 1, 2, c->nwin, c->stream))
    return -1;
  (void)N;
  bnh_qd_epi e = {p[5], p[6] == RT_F16, out, rt_ws(c, op, 1), p[7], p[8], p[9], (const float *)rt_b(c, op, 4),
                  rt_ws(c, op, 4)};
  return bnh_qd_gemm(a8, rt_ws(c, op, 2), Kp, rq, rt_ws(c, op, 3), 0, M, q, &e, c->nwin, c->stream);
}

// -------- SE_GATE16: b = [chsum f32 [C] (scaled to means in place), gate f16 [C]];
//          t = [reduce w [rd][C], reduce b [rd], expand w [C][rd], expand b [C]] (fp32); p = [C rd P]
//          (seg_init / seg_run, src/rt_ops_dot.c:352-420). The weights are held in fp16; the arithmetic is fp32.
void seg_fini(rt_op *op) { bnh_seg16_free((bnh_seg16 *)op->state); }
int seg_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 2, 4, 3)) return RT_E_PARAM;
  int C = op->p[0], rd = op->p[1];
  RT_REQ(c, op, C > 0 && C % 8 == 0 && rd > 0 && op->p[2] > 0);
  if (rt_need(c, op, 0, RT_F32, (size_t)C) || rt_need(c, op, 1, RT_F16, (size_t)C)) return RT_E_PARAM;
  if (need_f32_t(c, op, 0, (size_t)rd * C) || need_f32_t(c, op, 1, (size_t)rd) || need_f32_t(c, op, 2, (size_t)C * rd) ||
      need_f32_t(c, op, 3, (size_t)C))
    return RT_E_PARAM;
  bnh_seg16 *s = bnh_seg16_new(C, rd, (const float *)rt_t(c, op, 0, nullptr), (const float *)rt_t(c, op, 1, nullptr),
                               (const float *)rt_t(c, op, 2, nullptr), (const float *)rt_t(c, op, 3, nullptr));
  op->state = s;
  return s ? 0 : rt_oom(c, op, (size_t)4 * C * rd);
}
int seg_run(rt_ctx *c, rt_op *op) {
  return bnh_se_gate16((float *)rt_b(c, op, 0), rt_ws(c, op, 0), op->p[2], (const bnh_seg16 *)op->state,
                       (uint16_t *)rt_b(c, op, 1), rt_ws(c, op, 1), c->nwin, c->stream);
}

// -------- GEM_A: b = [F f32 [M][C], e f32 [C]]; t = [consts {eps, p}]; p = [M C]   (gem_init / gem_run,
//          src/rt_ops_dot.c:431-465): e[c] = (mean over rows of max(F, eps)^p)^(1/p)
int gem_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 2, 1, 2)) return RT_E_PARAM;
  int M = op->p[0], C = op->p[1];
  RT_REQ(c, op, M > 0 && C > 0 && C % 4 == 0);
  if (rt_need_rows(c, op, 0, RT_F32, (size_t)M, C) || rt_need(c, op, 1, RT_F32, (size_t)C) || need_f32_t(c, op, 0, 2))
    return RT_E_PARAM;
  return 0;
}
int gem_run(rt_ctx *c, rt_op *op) {
  const float *k = (const float *)rt_t(c, op, 0, nullptr);
  return bnh_gem_a((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), op->p[0], op->p[1], k[0], k[1],
                   (float *)rt_b(c, op, 1), rt_ws(c, op, 1), c->nwin, c->stream);
}

// -------- HEADS_S8: b = [F f32 [H*W][C], e f32 [C], logits f32 [ncp], a8 int8, rq f32];
//          t = [lin w [nc][C], lin b, then for the head over H and the head over W: fc w [hid][C], fc b, att w [nc][hid],
//               att b, cla w [nc][hid], cla b]; p = [H W C hid nc]   (heads_init / heads_run, src/rt_ops_dot.c:475-572)
struct hd_st {
  bnh_heads8 *P;
  void *work;
  size_t cap, ws;
};
void heads_fini(rt_op *op) {
  hd_st *s = (hd_st *)op->state;
  if (s) {
    bnh_heads8_free(s->P);
    if (s->work) bnh_free(s->work);
  }
  free(s);
}
int heads_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 5, 14, 5)) return RT_E_PARAM;
  const int *p = op->p;
  int H = p[0], W = p[1], C = p[2], hid = p[3], nc = p[4], ncp = (nc + 15) & ~15, L = H > W ? H : W;
  RT_REQ(c, op, H > 0 && W > 0 && C > 0 && C % 16 == 0 && hid > 0 && hid % 16 == 0 && nc > 0);
  int kq = C > hid ? C : hid;
  if (rt_need_rows(c, op, 0, RT_F32, (size_t)H * W, C) || rt_need(c, op, 1, RT_F32, (size_t)C) ||
      rt_need(c, op, 2, RT_F32, (size_t)ncp) || rt_need(c, op, 3, RT_I8, (size_t)(L + 4) * kq) ||
      rt_need(c, op, 4, RT_F32, (size_t)2 * (L + 4)))
    return RT_E_PARAM;
  if (need_f32_t(c, op, 0, (size_t)nc * C) || need_f32_t(c, op, 1, (size_t)nc)) return RT_E_PARAM;
  for (int i = 0; i < 2; i++) {
    int t = 2 + 6 * i;
    if (need_f32_t(c, op, t, (size_t)hid * C) || need_f32_t(c, op, t + 1, (size_t)hid) ||
        need_f32_t(c, op, t + 2, (size_t)nc * hid) || need_f32_t(c, op, t + 3, (size_t)nc) ||
        need_f32_t(c, op, t + 4, (size_t)nc * hid) || need_f32_t(c, op, t + 5, (size_t)nc))
      return RT_E_PARAM;
  }
  hd_st *s = (hd_st *)calloc(1, sizeof *s);
  op->state = s;
  if (!s) return rt_oom(c, op, sizeof *s);
  const float *w[7], *b[7];
  for (int i = 0; i < 7; i++) {
    w[i] = (const float *)rt_t(c, op, 2 * i, nullptr);
    b[i] = (const float *)rt_t(c, op, 2 * i + 1, nullptr);
  }
  s->ws = bnh_heads8_work_bytes(H, W, C, hid, nc);
  s->P = bnh_heads8_new(C, hid, nc, w, b);
  return s->P ? 0 : rt_oom(c, op, (size_t)ncp * kq * 7);
}
int heads_run(rt_ctx *c, rt_op *op) {
  hd_st *s = (hd_st *)op->state;
  const int *p = op->p;
  const size_t need = s->ws * (size_t)c->bcap;
  if (s->cap < need) {
    if (s->work) bnh_free(s->work);
    s->cap = 0;
    if (!(s->work = bnh_malloc(need))) {
      rt_oom(c, op, need);
      return -1;
    }
    s->cap = need;
  }
  return bnh_heads_s8((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), (const float *)rt_b(c, op, 1), rt_ws(c, op, 1),
                      p[0], p[1], s->P, (float *)rt_b(c, op, 2), rt_ws(c, op, 2), (int8_t *)rt_b(c, op, 3),
                      rt_ws(c, op, 3), (float *)rt_b(c, op, 4), rt_ws(c, op, 4), c->nwin,
                      (char *)s->work + s->ws * c->w0, s->ws, c->stream);  // this sub-batch's window slots
}

const rt_kernel K_STEM3 = {stem3_init, stem3_run, rt_dev_fini, "stem3_f32to16", 0x2, 0};
const rt_kernel K_PROTO8 = {bnh_proto8_dot_init, bnh_proto8_dot_run, bnh_proto8_dot_fini, "proto_s8", 0xe, 0};
const rt_kernel K_CONV3C24 = {c24_init, c24_run, c24_fini, "conv3c24_wino16", 0x2, 0};
const rt_kernel K_UNPAD = {unpad_init, unpad_run, nullptr, "unpad_f16to32", 0x2, 0};
const rt_kernel K_WINO_S8 = {wino_init, wino_run, wino_fini, "wino3_s8", 0x2, 0};
const rt_kernel K_QCONV3 = {qconv_init, qconv_run, qconv_fini, "qconv3_s8", 0x2, 0};
const rt_kernel K_QPW = {qpw_init, qpw_run, qw_fini, "qpw_s8", 0xe, 0x30};
const rt_kernel K_SE_GATE16 = {seg_init, seg_run, seg_fini, "se_gate16", 0x3, 0};
const rt_kernel K_GEM_A = {gem_init, gem_run, nullptr, "gem_a", 0x2, 0};
const rt_kernel K_HEADS_S8 = {heads_init, heads_run, heads_fini, "heads_s8", 0x1c, 0};

}  // namespace

const rt_kernel *rt_k_dot(int base) {
  switch (base) {
    case RT_OP_PROTO: return &K_PROTO8;  // the dotprod prototype head (src/rt_ops_f16.c:284-286)
    case RT_OP_STEM3: return &K_STEM3;
    case RT_OP_CONV3C24: return &K_CONV3C24;
    case RT_OP_UNPAD: return &K_UNPAD;
    case RT_OP_WINO_S8: return &K_WINO_S8;
    case RT_OP_QCONV3: return &K_QCONV3;
    case RT_OP_QPW: return &K_QPW;
    case RT_OP_SE_GATE16: return &K_SE_GATE16;
    case RT_OP_GEM_A: return &K_GEM_A;
    case RT_OP_HEADS_S8: return &K_HEADS_S8;
    default: return nullptr;
  }
}
