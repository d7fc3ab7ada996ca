// Registry kernels with fp32 arithmetic (variant 0 of the reference's rt_ops_f32.c family) on the GPU, plus the
// depthwise contract checks the fp16 family shares (as src/rt_ops_f32.c shares them with src/rt_ops_f16.c).
#include <stdlib.h>
#include <string.h>

#include "bnh_internal.h"
#include "rt.h"

// device copies of an op's first `n` tensors (weights / biases), freed by dev_fini
int rt_dev_tensors(rt_ctx *c, rt_op *op, int n) {
  rt_dev_state *s = (rt_dev_state *)calloc(1, sizeof *s);
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
  rt_dev_state *s = (rt_dev_state *)op->state;
  if (s) {
    for (int i = 0; i < 4; i++)
      if (s->t[i]) bnh_free(s->t[i]);
    if (s->scratch) bnh_free(s->scratch);
  }
  free(s);
}
void *rt_dev_scratch(rt_ctx *c, rt_op *op, size_t per_window) {
  rt_dev_state *s = (rt_dev_state *)op->state;
  const size_t want = per_window * (size_t)c->bcap;
  if (s->scratch_cap < want) {
    if (s->scratch) bnh_free(s->scratch);
    s->scratch_cap = 0;
    s->scratch = bnh_malloc(want);
    if (!s->scratch) {
      rt_oom(c, op, want);
      return nullptr;
    }
    s->scratch_cap = want;
  }
  return s->scratch;
}
static inline void *dev_tn(const rt_op *op, int i) { return ((rt_dev_state *)op->state)->t[i]; }

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

// the depthwise op computing its input itself: expansion op->pw's GEMM over the rows it quantized (bnh_pwdw_f32)
static int dw_fused_run(rt_ctx *c, rt_op *op, int k, int s, int pt, int pl, int form, int dact, int Ho, int Wo) {
  const rt_op *pw = op->pw;
  return bnh_pwdw_f32((const int8_t *)rt_b(c, pw, 3), rt_ws(c, pw, 3), (const float *)rt_b(c, pw, 4), rt_ws(c, pw, 4),
                      (const int32_t *)rt_b(c, pw, 5), rt_ws(c, pw, 5), op->p[0], op->p[1], rt_pw8_plain(pw),
                      pw->p[6], k, s, pt, pl, form, (const float *)dev_tn(op, 0), (const float *)dev_tn(op, 1), dact,
                      (float *)rt_b(c, op, 1), rt_ws(c, op, 1), Ho, Wo, (float *)rt_b(c, op, 2), rt_ws(c, op, 2),
                      c->nwin, c->stream);
}

static int dwk_init(rt_ctx *c, rt_op *op) {
  if (rt_dwk_check(c, op, 4)) return RT_E_PARAM;
  return rt_dev_tensors(c, op, 2);
}
static int dwk_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  if (op->pw) return dw_fused_run(c, op, p[3], p[4], p[5], p[6], 0, p[9], p[7], p[8]);
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
  if (op->pw) return dw_fused_run(c, op, 3, p[3], 1, 1, 2, 1, p[4], p[5]);
  return bnh_dw3_f32((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], p[2], p[3],
                     (const float *)dev_tn(op, 0), (const float *)dev_tn(op, 1), (float *)rt_b(c, op, 1),
                     rt_ws(c, op, 1), p[4], p[5], (float *)rt_b(c, op, 2), rt_ws(c, op, 2), c->nwin, c->stream);
}

// -------- FE_LOGMEL: b = [pcm, spec f32 [nfr][nmel]]; t = [window [frame], mel [nmel][nfft/2+1], consts {floor,
//          scale}]; p = [nsamp frame hop pad nfft nmel]   (src/rt_ops_f32.c:362-385)
static void logmel_fini(rt_op *op) { bnh_logmel_free((bnh_logmel *)op->state); }
static int logmel_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 2, 3, 6)) return RT_E_PARAM;
  const int *p = op->p;
  RT_REQ(c, op, p[0] > 0 && p[1] > 0 && p[2] > 0 && p[3] >= 0 && p[4] >= p[1] && p[5] > 0);
  if (rt_need_t(c, op, 0, (size_t)p[1] * 4, 0) || rt_need_t(c, op, 1, (size_t)p[5] * (p[4] / 2 + 1) * 4, 0) ||
      rt_need_t(c, op, 2, 8, 0))
    return RT_E_PARAM;
  if (rt_need(c, op, 0, RT_F32, (size_t)p[0]) || rt_need(c, op, 1, RT_F32, 1)) return RT_E_PARAM;
  RT_REQ(c, op, (p[4] & (p[4] - 1)) == 0 && p[4] >= 16 && p[4] <= 2048);  // nfft
  RT_REQ(c, op, p[1] <= p[4] && p[5] <= 512);                             // frame, nmel
  const float *k = (const float *)rt_t(c, op, 2, nullptr);
  bnh_logmel *F = bnh_logmel_new(p[0], p[1], p[2], p[3], p[4], p[5], (const float *)rt_t(c, op, 0, nullptr),
                                 (const float *)rt_t(c, op, 1, nullptr), k[0], k[1]);
  op->state = F;
  if (!F) return rt_oom(c, op, (size_t)p[4] * 16);
  return rt_need(c, op, 1, RT_F32, (size_t)bnh_logmel_frames(F) * p[5]);
}
static int logmel_run(rt_ctx *c, rt_op *op) {
  return bnh_logmel_run((const bnh_logmel *)op->state, (const float *)rt_b(c, op, 0), rt_ws(c, op, 0),
                        (float *)rt_b(c, op, 1), rt_ws(c, op, 1), c->nwin, c->stream);
}

// -------- STEM: b = [img f32 [H][W], out, col]; t = [w panels [Np/8][Kp][8], b]; p = [N K Kp Np, H W Ho Wo k s act
//          ldo opad]   (rt_stem_f32_check, src/rt_ops_f32.c:390-415). The im2col buffer (b[2]) is not used: the
//          kernel reads the taps from the image directly.
// rt_stem_f32_check (src/rt_ops_f32.c:390-408), shared with the fp16 path's STEM
int rt_stem_check(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, -1, 2, 13)) return RT_E_PARAM;
  const int *p = op->p;
  const int N = p[0], K = p[1], Kp = p[2], Np = p[3];
  if (N <= 0 || K <= 0 || Np != ((N + 7) & ~7) || Kp < K || Kp % 4)
    return rt_bad(c, op, "GEMM shape N %d K %d Kp %d Np %d: expected Np = N rounded up to 8, Kp >= K, Kp %% 4 == 0", N,
                  K, Kp, Np);
  if (rt_need_t(c, op, 0, (size_t)Np * Kp * 4, 1) || rt_need_t(c, op, 1, (size_t)Np * 4, 1)) return RT_E_PARAM;
  const int H = p[4], W = p[5], Ho = p[6], Wo = p[7], k = p[8], s = p[9], ldo = p[11], h = p[12];
  RT_REQ(c, op, k >= 1 && s >= 1 && Ho > 0 && Wo > 0);
  RT_REQ(c, op, (Ho - 1) * s + k <= H && (Wo - 1) * s + k <= W);  // VALID conv
  RT_REQ(c, op, K == k * k);
  RT_REQ(c, op, ldo >= Np);  // the GEMM stores whole 8-channel panels
  RT_REQ(c, op, h >= 0 && h <= 3);
  RT_REQ(c, op, p[10] >= 0 && p[10] <= 2);
  if (rt_need(c, op, 0, RT_F32, (size_t)H * W) || rt_need(c, op, 2, RT_F32, (size_t)((Ho * Wo + 7) & ~7) * Kp))
    return RT_E_PARAM;
  const rt_bufdesc *o = rt_bd(c, op, 1);
  if (!o) return rt_bad(c, op, "buffer argument 1 (output) is absent");
  if (o->halo != (uint32_t)h || o->ld != (uint32_t)ldo || (h && (o->W != (uint32_t)Wo || o->H != (uint32_t)Ho)))
    return rt_bad(c, op, "buffer argument 1 (buffer #%d, output): expected %d x %d, halo %d, ld %d; found %u x %u, halo "
                  "%u, ld %u", op->b[1], Ho, Wo, h, ldo, o->H, o->W, o->halo, o->ld);
  if (rt_need(c, op, 1, (int)o->dtype, (size_t)(Ho + 2 * h) * (Wo + 2 * h) * ldo)) return RT_E_PARAM;
  return rt_dev_tensors(c, op, 2);
}
static int stem_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 3, -1, -1) || rt_stem_check(c, op) || rt_need(c, op, 1, RT_F32, 1)) return RT_E_PARAM;
  RT_REQ(c, op, op->p[11] % 4 == 0);  // 4-channel output groups
  return 0;
}
static int stem_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  if (p[12] && !rt_halo_kept(c, op, 1) &&
      bnh_zero_halo(rt_b(c, op, 1), rt_ws(c, op, 1), p[6], p[7], p[11], p[12], 4, c->nwin, c->stream))
    return -1;
  return bnh_stem_f32_body((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[4], p[5], p[8], p[9], p[6], p[7],
                           (const float *)dev_tn(op, 0), (const float *)dev_tn(op, 1), p[2], p[3], p[10],
                           (float *)rt_b(c, op, 1), rt_ws(c, op, 1), p[11], p[12], c->nwin, c->stream);
}

// -------- PW: b = [in f32 [M][lda], out, res | -1 (, gate f32 [K] | -1)]; t = [w panels [Np/8][Kp][8], b];
//          p = [N K Kp Np, M, lda, act, ldo, ow, opad, ldr]   (pw_init / rt_pw_check / rt_fpack_view,
//          src/rt_ops_f32.c:49-59, 129-162; pw_run :194-208)
int rt_pw_out_check(rt_ctx *c, rt_op *op, int dt);  // ops_s8n.cpp
static int pw_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, op->nb == 4 ? 4 : 3, 2, 11)) return RT_E_PARAM;  // the gate is optional
  const int *p = op->p;
  const int N = p[0], K = p[1], Kp = p[2], Np = p[3];
  if (N <= 0 || K <= 0 || Np != ((N + 7) & ~7) || Kp < K || Kp % 4)
    return rt_bad(c, op, "GEMM shape N %d K %d Kp %d Np %d: expected Np = N rounded up to 8, Kp >= K, Kp %% 4 == 0", N,
                  K, Kp, Np);
  if (rt_need_t(c, op, 0, (size_t)Np * Kp * 4, 1) || rt_need_t(c, op, 1, (size_t)Np * 4, 1)) return RT_E_PARAM;
  if (op->nb == 4 && op->b[3] >= 0) {
    RT_REQ(c, op, K == Kp);
    if (rt_need(c, op, 3, RT_F32, (size_t)K)) return RT_E_PARAM;
  }
  const int M = p[4], lda = p[5], act = p[6], ldo = p[7], opad = p[9], ldr = p[10];
  const size_t Mr = ((size_t)M + 7) & ~(size_t)7;
  RT_REQ(c, op, M > 0);
  RT_REQ(c, op, lda >= Kp);  // the input channel stride covers the packed K
  RT_REQ(c, op, ldo >= Np);  // the output channel stride covers the packed N
  RT_REQ(c, op, act >= 0 && act <= 2);
  RT_REQ(c, op, opad >= 0 && opad <= 3);
  if (rt_need(c, op, 0, RT_F32, Mr * lda) || rt_pw_out_check(c, op, RT_F32)) return RT_E_PARAM;  // 8-row tiles
  if (op->b[2] >= 0) {
    RT_REQ(c, op, ldr >= Np);
    const rt_bufdesc *r = rt_bd(c, op, 2);
    if (r->halo) {  // a residual in a zero-haloed buffer: the same pixel grid as the M rows
      if (r->dtype != RT_F32 || r->ld != (uint32_t)ldr || (size_t)r->H * r->W != (size_t)M || !r->W)
        return rt_bad(c, op, "buffer argument 2 (buffer #%d, residual): halo %u needs an fp32 buffer with ld %d and H x W = "
                      "%d rows, found %s ld %u %ux%u", op->b[2], r->halo, ldr, M, rt_dtype_name(r->dtype), r->ld, r->H, r->W);
      if (rt_need(c, op, 2, RT_F32, (size_t)(r->H + 2 * r->halo) * (r->W + 2 * r->halo) * ldr)) return RT_E_PARAM;
    } else if (rt_need(c, op, 2, RT_F32, (size_t)M * ldr)) {
      return RT_E_PARAM;
    }
  }
  return rt_dev_tensors(c, op, 2);
}
static int pw_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  const rt_bufdesc *r = rt_bd(c, op, 2);
  const bool gated = op->nb == 4 && op->b[3] >= 0;
  bnh_epi32 e = {p[6], (float *)rt_b(c, op, 1), rt_ws(c, op, 1), p[7], p[9] ? p[8] : 0, p[9],
                 (const float *)rt_b(c, op, 2), rt_ws(c, op, 2), p[10], r ? (int)r->halo : 0, r ? (int)r->W : 0};
  if (e.opad && !rt_halo_kept(c, op, 1) &&
      bnh_zero_halo(e.out, e.out_ws, p[4] / p[8], p[8], p[7], p[9], 4, c->nwin, c->stream))
    return -1;
  return bnh_gemm_f32((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[5], p[4],
                      gated ? (const float *)rt_b(c, op, 3) : nullptr, gated ? rt_ws(c, op, 3) : 0,
                      (const float *)dev_tn(op, 0), (const float *)dev_tn(op, 1), p[2], p[3], &e, c->nwin, c->stream);
}

// -------- SE / SE_GATE: SE b = [D [P][C], chsum]; SE_GATE b = [chsum, gate f32 [C]]; t = [w1 [rd][C], b1 [rd],
//          w2t [rd][C], b2 [C]]; p = [C rd P]   (rt_se_check, src/rt_ops_f32.c:256-266)
static int se_check(rt_ctx *c, rt_op *op, int gate) {
  if (rt_need_args(c, op, 2, 4, 3)) return RT_E_PARAM;
  const int C = op->p[0], rd = op->p[1], P = op->p[2];
  RT_REQ(c, op, C > 0 && C % 8 == 0 && C <= 4096);
  RT_REQ(c, op, rd > 0 && rd <= 512);
  RT_REQ(c, op, P > 0);
  const size_t want[4] = {(size_t)rd * C, (size_t)rd, (size_t)rd * C, (size_t)C};
  for (int i = 0; i < 4; i++)
    if (rt_need_t(c, op, i, want[i] * 4, 0)) return RT_E_PARAM;
  if (rt_need(c, op, 0, RT_F32, gate ? (size_t)C : (size_t)P * C) || rt_need(c, op, 1, RT_F32, (size_t)C))
    return RT_E_PARAM;
  return rt_dev_tensors(c, op, 4);
}
static int se_init(rt_ctx *c, rt_op *op) { return se_check(c, op, 0); }
static int seg_init(rt_ctx *c, rt_op *op) { return se_check(c, op, 1); }
static int se_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  // op scratch per window: the gates (16-byte aligned rows), then the first FC's outputs
  const long long g_ws = (p[0] + 3) / 4 * 4;
  float *g = (float *)rt_dev_scratch(c, op, sizeof(float) * (size_t)(g_ws + p[1]));
  if (!g) return -1;
  return bnh_se_f32((const float *)rt_b(c, op, 1), rt_ws(c, op, 1), p[0], p[1], p[2], (const float *)dev_tn(op, 0),
                    (const float *)dev_tn(op, 1), (const float *)dev_tn(op, 2), (const float *)dev_tn(op, 3),
                    g + g_ws * c->w0, g_ws, g + g_ws * c->bcap + (long long)p[1] * c->w0, (float *)rt_b(c, op, 0),
                    rt_ws(c, op, 0), c->nwin, c->stream);
}
static int seg_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  float *work = (float *)rt_dev_scratch(c, op, sizeof(float) * (size_t)p[1]);  // the first FC's outputs
  if (!work) return -1;
  return bnh_se_f32((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], p[2], (const float *)dev_tn(op, 0),
                    (const float *)dev_tn(op, 1), (const float *)dev_tn(op, 2), (const float *)dev_tn(op, 3),
                    (float *)rt_b(c, op, 1), rt_ws(c, op, 1), work + (long long)p[1] * c->w0, nullptr, 0, c->nwin,
                    c->stream);
}

// -------- MEAN: b = [x [P][ld], out f32 [C]]; p = [P C ld]   (rt_mean_check, src/rt_ops_f32.c:510-522)
int rt_mean_check(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 2, -1, 3)) return RT_E_PARAM;
  RT_REQ(c, op, op->p[0] > 0 && op->p[1] > 0);
  RT_REQ(c, op, op->p[1] % 4 == 0);
  RT_REQ(c, op, op->p[2] >= op->p[1]);
  const rt_bufdesc *x = rt_bd(c, op, 0);
  if (!x) return rt_bad(c, op, "buffer argument 0 (input) is absent");
  if (x->halo)
    return rt_bad(c, op, "buffer argument 0 (buffer #%d, input): expected no halo, found halo %u", op->b[0], x->halo);
  if (rt_need(c, op, 0, (int)x->dtype, (size_t)op->p[0] * op->p[2]) || rt_need(c, op, 1, RT_F32, (size_t)op->p[1]))
    return RT_E_PARAM;
  return 0;
}
static int mean_init(rt_ctx *c, rt_op *op) {
  return rt_mean_check(c, op) || rt_need(c, op, 0, RT_F32, 1) ? RT_E_PARAM : 0;
}
static int mean_run(rt_ctx *c, rt_op *op) {
  return bnh_mean_f32((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), op->p[0], op->p[1], op->p[2],
                      (float *)rt_b(c, op, 1), rt_ws(c, op, 1), c->nwin, c->stream);
}

// -------- PAD: b = [x, xp (halo h)]; p = [H W C ld h]   (rt_pad_check, src/rt_ops_f32.c:480-501)
int rt_pad_check(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 2, -1, 5)) return RT_E_PARAM;
  const int *p = op->p;
  const rt_bufdesc *x = rt_bd(c, op, 0), *o = rt_bd(c, op, 1);
  if (!x || !o) return rt_bad(c, op, "buffer argument %d is absent", x ? 1 : 0);
  RT_REQ(c, op, p[0] > 0 && p[1] > 0 && p[2] > 0);
  RT_REQ(c, op, p[4] >= 1 && p[4] <= 3);
  RT_REQ(c, op, p[3] >= p[2]);
  if (x->dtype != o->dtype)
    return rt_bad(c, op, "buffer argument 0 (buffer #%d, input) is %s but buffer argument 1 (buffer #%d, output) is %s",
                  op->b[0], rt_dtype_name(x->dtype), op->b[1], rt_dtype_name(o->dtype));
  if (x->halo)
    return rt_bad(c, op, "buffer argument 0 (buffer #%d, input): expected no halo, found halo %u", op->b[0], x->halo);
  if (o->ld != (uint32_t)p[2] || o->halo != (uint32_t)p[4])
    return rt_bad(c, op, "buffer argument 1 (buffer #%d, output): expected ld %d halo %d, found ld %u halo %u", op->b[1],
                  p[2], p[4], o->ld, o->halo);
  if (rt_need(c, op, 0, (int)x->dtype, (size_t)p[0] * p[1] * p[3]) ||
      rt_need(c, op, 1, (int)o->dtype, (size_t)(p[0] + 2 * p[4]) * (p[1] + 2 * p[4]) * p[2]))
    return RT_E_PARAM;
  return 0;
}
static int pad_init(rt_ctx *c, rt_op *op) {
  return rt_pad_check(c, op) || rt_need(c, op, 0, RT_F32, 1) ? RT_E_PARAM : 0;
}
int rt_pad_run(rt_ctx *c, rt_op *op, int esz) {
  const int *p = op->p;
  return bnh_pad(rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], p[2], p[3], p[4], esz, rt_b(c, op, 1), rt_ws(c, op, 1),
                 c->nwin, c->stream);
}
static int pad_run(rt_ctx *c, rt_op *op) { return rt_pad_run(c, op, 4); }

// -------- GEMV: b = [x f32 [K], out f32 [N]]; t = [w [N][K] (fp32; fp16 in the fp16 path), b f32 [N]];
//          p = [N K act]   (rt_gemv_check, src/rt_ops_f32.c:593-601)
int rt_gemv_check(rt_ctx *c, rt_op *op, size_t esz) {
  if (rt_need_args(c, op, 2, 2, 3)) return RT_E_PARAM;
  const int N = op->p[0], K = op->p[1];
  RT_REQ(c, op, N > 0 && K > 0);
  RT_REQ(c, op, op->p[2] == 0 || op->p[2] == 2);
  if (rt_need_t(c, op, 0, (size_t)N * K * esz, 0) || rt_need_t(c, op, 1, (size_t)N * 4, 0)) return RT_E_PARAM;
  if (rt_need(c, op, 0, RT_F32, (size_t)K) || rt_need(c, op, 1, RT_F32, (size_t)N)) return RT_E_PARAM;
  RT_REQ(c, op, (size_t)K * 4 <= 64 * 1024);  // one window's input in LDS
  return rt_dev_tensors(c, op, 2);
}
static int gemv_init(rt_ctx *c, rt_op *op) { return rt_gemv_check(c, op, 4); }
int rt_gemv_run(rt_ctx *c, rt_op *op, int w16) {
  return bnh_gemv(dev_tn(op, 0), w16, (const float *)dev_tn(op, 1), op->p[0], op->p[1], (const float *)rt_b(c, op, 0),
                  rt_ws(c, op, 0), op->p[2], (float *)rt_b(c, op, 1), rt_ws(c, op, 1), c->nwin, c->stream);
}
static int gemv_run(rt_ctx *c, rt_op *op) { return rt_gemv_run(c, op, 0); }
void *rt_dev_t(const rt_op *op, int i) { return dev_tn(op, i); }

static const rt_kernel K_GEMV = {gemv_init, gemv_run, rt_dev_fini, "gemv_f32", 0x2, 0};
static const rt_kernel K_PW = {pw_init, pw_run, rt_dev_fini, "pw_f32", 0x2, 0xc};
static const rt_kernel K_LOGMEL = {logmel_init, logmel_run, logmel_fini, "fe_logmel", 0x2, 0};
static const rt_kernel K_STEM = {stem_init, stem_run, rt_dev_fini, "stem_f32", 0x6, 0};
static const rt_kernel K_SE = {se_init, se_run, rt_dev_fini, "se_f32", 0x1, 0};
static const rt_kernel K_SE_GATE = {seg_init, seg_run, rt_dev_fini, "se_gate_f32", 0x2, 0};
static const rt_kernel K_MEAN = {mean_init, mean_run, nullptr, "mean_f32", 0x2, 0};
static const rt_kernel K_PAD = {pad_init, pad_run, nullptr, "pad_f32", 0x2, 0};
static const rt_kernel K_DW3 = {dw3_init, dw3_run, rt_dev_fini, "dw3_f32", 0x6, 0};
static const rt_kernel K_DWK = {dwk_init, dwk_run, rt_dev_fini, "dwk_f32", 0x6, 0};

int rt_fuse_pwdw(rt_ctx *c, rt_op *pw, rt_op *dw) {
  (void)c;
  const bnh_s8w *W = rt_pw8_plain(pw);
  if (!W || (dw->k != &K_DW3 && dw->k != &K_DWK) || dw->b[0] != pw->b[1]) return 0;
  const int *p = pw->p, *d = dw->p;
  const bool dw3 = dw->k == &K_DW3;
  const int H = d[0], Wd = d[1], C = d[2];
  const int k = dw3 ? 3 : d[3], s = dw3 ? d[3] : d[4], pt = dw3 ? 1 : d[5], pl = dw3 ? 1 : d[6];
  const int Ho = dw3 ? d[4] : d[7], Wo = dw3 ? d[5] : d[8];
  // the expansion fills exactly the depthwise input: C channels of H x W pixels, halo (k - 1) / 2
  if (p[3] != C || p[7] != C || p[4] != H * Wd || p[8] != Wd || p[9] != (k - 1) / 2) return 0;
  if (bnh_pwdw_f32_plan(C, p[2], H, Wd, k, s, pt, pl, dw3 ? 2 : 0, Ho, Wo)) {
    bnh_clear_error();
    return 0;
  }
  pw->quant_only = 1;
  dw->pw = pw;
  return 1;
}

// the fp32 prototype heads (ops_proto.cpp)
int bnh_proto_f32_init(rt_ctx *c, rt_op *op);
int bnh_proto_f32h_init(rt_ctx *c, rt_op *op);
int bnh_proto_fp_run(rt_ctx *c, rt_op *op);
void bnh_proto_fp_fini(rt_op *op);
static const rt_kernel K_PROTO = {bnh_proto_f32_init, bnh_proto_fp_run, bnh_proto_fp_fini, "proto_f32", 0xe, 0};
static const rt_kernel K_PROTO_F32H = {bnh_proto_f32h_init, bnh_proto_fp_run, bnh_proto_fp_fini, "proto_f32h", 0xe, 0};

const rt_kernel *rt_k_f32(int base) {
  switch (base) {
    case RT_OP_PROTO: return &K_PROTO;
    case RT_OP_PROTO_F32H: return &K_PROTO_F32H;
    case RT_OP_PW: return &K_PW;
    case RT_OP_DW3: return &K_DW3;
    case RT_OP_DWK: return &K_DWK;
    case RT_OP_FE_LOGMEL: return &K_LOGMEL;
    case RT_OP_STEM: return &K_STEM;
    case RT_OP_SE: return &K_SE;
    case RT_OP_SE_GATE: return &K_SE_GATE;
    case RT_OP_MEAN: return &K_MEAN;
    case RT_OP_PAD: return &K_PAD;
    case RT_OP_GEMV: return &K_GEMV;
    default: return nullptr;
  }
}
