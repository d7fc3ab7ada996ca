/* CPU oracle for the quantized conv/GEMM hot path of libbnneon (cdw9bf/birdnet-neon-engine).
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker (or as the timed CPU baseline). The product path (libbnneon_hip.so) never links,
 * loads or calls it.
 *
 * Every function restates, in scalar C, what the reference's NEON kernels compute, element by element, with the
 * AArch64 floating-point semantics those kernels run under (FPCR default: round to nearest even, no flush to zero,
 * NaN-propagating FMIN/FMAX, saturating float->int conversions, FRECPE/FRECPS as in the Arm ARM pseudocode). Build
 * flags: -O2 -ffp-contract=off (the reference's Makefile:16), so every a*b+c below is two roundings unless it is an
 * explicit fmaf. Each function names the reference file:line it follows.
 *
 * Where the reference has no kernel (the Q31 requantised GEMM, the int8 depthwise) the function is this project's own
 * written specification; its header comment says so.
 */
#ifndef BNN_ORACLE_H
#define BNN_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- AArch64 scalar semantics */
float orc_frecpe(float x);                 /* FRECPE (Arm ARM FPRecipEstimate, FPCR.FZ = 0, RN) */
float orc_frecps(float a, float b);        /* FRECPS: 2 - a*b fused, with the (inf, 0) -> 2 rule */
float orc_fmax(float a, float b);          /* FMAX: NaN-propagating, +0 > -0 */
float orc_fmin(float a, float b);          /* FMIN: NaN-propagating, -0 < +0 */
int32_t orc_cvtn_s32(float x);             /* FCVTNS w: round to nearest even, saturating, NaN -> 0 */
int32_t orc_cvta_s32(float x);             /* FCVTAS w: round to nearest ties away, saturating, NaN -> 0 */
int32_t orc_lrintf_s32(float x);           /* (int32_t)lrintf(x) on AArch64: FRINTX + FCVTZS x, low 32 bits */
float orc_silu_f32(float x);               /* silu_f32x4 / silu4_f32x4 lane (src/gemm_f32.h:102-145) */
void orc_eval_f32(int f, const float *x, float *y, long long n); /* 0 FRECPE, 1 SiLU, 2 ReLU, elementwise */

/* ---------------------------------------------------------------- int8 no-dotprod GEMM (PW_S8) */
typedef struct {
  int act;          /* 0 none, 1 SiLU, 2 ReLU (src/gemm_f32.h:14) */
  float *out;
  int ldo, ow, opad;
  const float *res;
  int ldr, rpad, rw;
} orc_epi32;        /* src/gemm_f32.h:15-24 */

/* src/gemm_s8n.c:15-51 */
void orc_s8n_quant_rows(const float *x, int ld, int r0, int r1, int K, int Kp, int8_t *q, float *sa, int32_t *za);
/* src/gemm_s8n.c:55-63 */
void orc_s8n_quant_rows_gate(const float *x, int ld, int r0, int r1, int K, int Kp, const float *gate, int8_t *q,
                             float *sa, int32_t *za);
/* src/gemm_s8n.c:82-190: every row m < M and channel n < Np of act(dequant(q . W) + b) (+ residual), stored by the
 * epi32 rules. w is the package layout [Np/4][Kp/16][4][16]. */
void orc_s8n_gemm(const int8_t *q, int Kp, const float *sa, const int32_t *za, int M, int Np, const int8_t *w,
                  const float *sw, const int32_t *colsum, const float *b, const orc_epi32 *e);
/* the PW_S8 op of one window (src/rt_ops_s8n.c:119-134): halo zeroing of a padded output (H = M / ow rows), the
 * quantization of rows [0, M) and the GEMM */
void orc_pw_s8(const float *in, int lda, int M, int K, int Kp, int N, int Np, const float *gate, int8_t *q, float *sa,
               int32_t *za, const int8_t *w, const float *sw, const int32_t *colsum, const float *b, const orc_epi32 *e);
/* rt_zero_halo (src/rt_pkg.c:194-203) */
void orc_zero_halo(void *xp, int H, int W, int C, int h, size_t esz);

/* ---------------------------------------------------------------- int8 prototype head (PROTO_S8) */
/* src/proto_s8n.c:28-51 */
void orc_quant_cells_f32(const float *x, int P, int C, int ld, float eps, int8_t *qa, int Kp, float *sx);
/* src/proto_s8n.c:115-132 */
int orc_proto_n4_check(const int8_t *qw, int Kp, const uint8_t *n4, int npanels);
/* src/proto_s8n.c:139-164, every panel: prototypes [Np/4][Kp/16][4][16] */
void orc_proto_colmax_s8n(const int8_t *qa, int Kp, const float *sx, int P, const int8_t *qw, const float *sw, int Np,
                          float *colmax);
/* src/pc_kern_f32.c:364-374 */
int orc_proto_logits(const float *colmax, const float *w, const float *b, int nc, int ppc, float *logits);
/* the whole op of one window: quantize, column maxima, logits (src/rt_ops_s8n.c:245-253); returns 0 or -2 */
int orc_proto_s8(const float *x, int P, int C, int ld, float eps, int8_t *qa, int Kp, float *sx, const int8_t *qw,
                 const float *sw, int Np, float *colmax, const float *clsw, const float *clsb, int nc, int ppc,
                 float *logits);
/* ---------------------------------------------------------------- fp32 / fp16 prototype heads */
/* src/pc_kern_f32.c:350-362 */
void orc_l2norm_f32(const float *x, int P, int C, int ld, float eps, float *a);
/* src/pc_kern_f16.c:123-140 */
void orc_l2norm_f16(const uint16_t *x, int P, int C, int ld, float eps, uint16_t *a);
/* src/gemm_f32.c:443-460: fp32 panels [Np/8][Kp][8] */
void orc_colmax_f32(const float *A, int lda, int M, const float *wp, int Kp, int Np, float *colmax);
/* src/pc_kern_f32.c:378-407: fp16 panels [Np/8][K][8] */
void orc_colmax_f32h(const float *a, int P, int K, const uint16_t *w16, int Np, float *colmax);
/* src/gemm_f16.c:210-253: hpack panels [Np/16][Kp][16] + tail [Kp][8] */
void orc_colmax_f16(const uint16_t *A, int lda, int M, const uint16_t *W, int Kp, int Np, float *colmax);
/* PROTO variant 0 (src/rt_ops_f32.c:563-570), PROTO_F32H (:583-590), PROTO variant 1 (src/rt_ops_f16.c:236-250) */
int orc_proto_f32(const float *x, int P, int C, int ld, float eps, float *a, const float *wp, int Np, float *colmax,
                  const float *clsw, const float *clsb, int nc, int ppc, float *logits);
int orc_proto_f32h(const float *x, int P, int C, int ld, float eps, float *a, const uint16_t *w16, int Np,
                   float *colmax, const float *clsw, const float *clsb, int nc, int ppc, float *logits);
int orc_proto_f16(const uint16_t *x, int P, int C, int ld, float eps, uint16_t *a, const uint16_t *W, int Np,
                  float *colmax, const float *clsw, const float *clsb, int nc, int ppc, float *logits);


/* ---------------------------------------------------------------- depthwise convolutions */
/* fp16 values as bit patterns; one rounding to nearest even per operation, denormals kept */
float orc_h2f(uint16_t h);
uint16_t orc_h_fma(uint16_t a, uint16_t b, uint16_t c);   /* a * b + c */
uint16_t orc_h_add(uint16_t a, uint16_t b);
uint16_t orc_h_mul(uint16_t a, uint16_t b);
uint16_t orc_silu_lut_h(uint16_t x);                       /* src/silu_lut.h:28-42 */
/* src/pc_kern_f32.c:163-334 (DWK fp32) */
void orc_dwk_f32(const float *xp, int H, int W, int C, int k, int s, int pt, int pl, const float *w, const float *b,
                 int act, float *out, int Ho, int Wo, float *chsum);
/* src/gemm_f32.c:213-441 (DW3 fp32: pads 1, SiLU) */
void orc_dw3_f32(const float *xp, int H, int W, int C, int s, const float *w, const float *b, float *out, int Ho,
                 int Wo, float *chsum);
/* src/pc_kern_f16.c:16-96 (DWK fp16) */
void orc_dwk_f16(const uint16_t *xp, int H, int W, int C, int k, int s, int pt, int pl, const uint16_t *w,
                 const uint16_t *b, int act, uint16_t *out, int Ho, int Wo, float *chsum);
/* src/kern_f16.c:83-155 (DW3 fp16: SiLU) */
void orc_dw3_f16(const uint16_t *xp, int H, int W, int C, int s, int pt, int pl, const uint16_t *w, const uint16_t *b,
                 uint16_t *out, int Ho, int Wo, float *chsum);
/* int8 depthwise: this project's own specification (no reference kernel); dw.c states it */
void orc_dw_s8(const int8_t *x, int H, int W, int C, int k, int s, int pt, int pl, const int8_t *w, const int32_t *bias,
               const int32_t *mult, const int32_t *shift, int zx, int zy, int lo, int hi, const int8_t *lut, int8_t *out,
               int Ho, int Wo);

/* ---------------------------------------------------------------- fp16 GEMM (PW f16) */
uint16_t orc_f2h(float f);                                 /* FCVT h, s: nearest even, denormals, overflow to inf */
uint16_t orc_h_max(uint16_t a, uint16_t b);                /* FMAX on fp16 */
typedef struct {
  int act;          /* 0 none, 1 SiLU (LUT), 2 ReLU (src/gemm_f16.h:18) */
  uint16_t *out;
  int ldo, ow, opad;
  const uint16_t *res;
  int ldr;
} orc_epi16;        /* src/gemm_f16.h:19-27 (without the pooled form) */
/* src/gemm_f16.c:49-171: out rows [0, M) x channels [0, Np) of act(A . W^T + b) (+ res); W [N][Kp] channel rows, fp16
 * accumulation in balanced K blocks of <= 128 steps, fp32 across blocks */
void orc_gemm_f16(const uint16_t *A, int lda, int M, const uint16_t *W, int N, int Kp, const float *b32,
                  const uint16_t *b16, const orc_epi16 *e);

/* ---------------------------------------------------------------- int8 Winograd F(2x2,3x3) (WINO_S8) */
int32_t orc_cvtz_s32(float x);  /* FCVTZS w: toward zero, saturating, NaN -> 0 */
/* src/wino.c:26-88: w OHWI fp32 [K][3][3][C] -> U8 [16][K][C], sw [K], zw [4][K] */
void orc_wino8_pack(const float *w, int K, int C, int8_t *U8, float *sw, float *zw);
/* src/wino.c:117-227 for one window: x f32 [H][W][C] -> out fp16 [H][W][K] (bias, LUT SiLU) */
void orc_wino8(const float *x, int H, int W, int C, int K, const int8_t *U8, const float *sw, const float *zw,
               const float *bias, uint16_t *out);

/* ---------------------------------------------------------------- fp16 Winograd, 24 channels (CONV3C24) */
int orc_recip_estimate(int a);                    /* Arm ARM RecipEstimate on the 9-bit scaled operand */
uint16_t orc_h_min(uint16_t a, uint16_t b);       /* FMIN on fp16 */
uint16_t orc_frecpe_h(uint16_t x);                /* FRECPE, half precision */
uint16_t orc_frecps_h(uint16_t a, uint16_t b);    /* FRECPS, half precision */
uint16_t orc_silu_poly_h(uint16_t x);             /* silu4w, src/wino_s0.c:14-34 */
/* src/wino_s0.c:40-64: w OHWI fp32 [24][3][3][24] -> U fp16 [16][24 ci][24 co], b16 [24] */
void orc_wino_s0_pack(const float *w, const float *bias, uint16_t *U, uint16_t *b16);
/* src/wino_s0.c:145-165 over all tile rows: x, out padded fp16 [H+2][W+2][24]; out = SiLU(conv + b) + x */
void orc_wino_s0(const uint16_t *x, int H, int W, const uint16_t *U, const uint16_t *b16, uint16_t *out);

/* ---------------------------------------------------------------- Q31 requantised int8 GEMM (own specification)
 * The reference has no such kernel. Specification (TFLite / gemmlowp fixed-point conventions):
 *   acc[n][m]  = sum_k w[n][k] * (x[k][m] - zx) + bias[n]                       (exact, int32)
 *   y          = RoundingDivideByPOT(SaturatingRoundingDoublingHighMul(acc, mult[n]), shift[n]) + zy
 *   out[n][m]  = clamp(y, lo, hi)                                               (int8)
 * w int8 [N][K] row-major; x int8 [K][M] (NCHW: pixels contiguous); out int8 [N][M]. */
int32_t orc_srdhm(int32_t a, int32_t b);
int32_t orc_rdbypot(int32_t x, int exponent);
int8_t orc_requant(int32_t acc, int32_t mult, int shift, int zy, int lo, int hi);
void orc_gemm_s8_requant(const int8_t *w, const int8_t *x, const int32_t *bias, const int32_t *mult, const int32_t *shift,
                         int N, int K, int M, int zx, int zy, int lo, int hi, int8_t *out);

/* ---------------------------------------------------------------- fp32 ops around the int8 GEMMs (fe.c) */
float orc_log2_acc(float x);                      /* log2_acc_f32x4 lane, src/gemm_f32.h:57-71 */
float orc_exp2_f32(float t);                      /* exp2_f32x4 lane, src/gemm_f32.h:74-85 */
float orc_sigmoid_f32(float x);                   /* sigmoid_f32x4 lane, src/gemm_f32.h:93-96 */
int orc_logmel_frames(int nsamp, int frame, int hop, int pad);
/* FE_LOGMEL of one window (src/pc_kern_f32.c:28-149): spec [nfr][nmel]; returns nfr, or -1 for refused limits */
int orc_logmel(const float *pcm, int nsamp, int frame, int hop, int pad, int nfft, int nmel, const float *window,
               const float *mel, float floor_, float scale, float *spec);
/* gemm_f32 (src/gemm_f32.c:141-197), w [Np/8][Kp][8], optional input gate */
void orc_gemm_f32(const float *A, int lda, int M, const float *w, const float *b, int Kp, int Np, const float *gate,
                  const orc_epi32 *e);
/* STEM (src/rt_ops_f32.c:416-425): im2col of a 1-channel image, VALID k x k stride s, then gemm_f32 */
void orc_stem_f32(const float *img, int H, int W, int k, int s, int Ho, int Wo, const float *w, const float *b, int Kp,
                  int Np, const orc_epi32 *e);
/* SE_GATE (src/rt_ops_f32.c:317-324): gate [C] from the channel sums of P pixels */
void orc_se_gate_f32(const float *chsum, int C, int rd, int P, const float *w1, const float *b1, const float *w2t,
                     const float *b2, float *gate);
/* SE (src/rt_ops_f32.c:297-309): D [P][C] gated in place */
void orc_se_f32(float *D, int P, int C, const float *chsum, int rd, const float *w1, const float *b1, const float *w2t,
                const float *b2);
void orc_mean_f32(const float *x, int P, int C, int ld, float *out);  /* src/pc_kern_f32.c:342-348 */
void orc_pad(const void *x, int H, int W, int C, int ld, int h, size_t esz, void *xp);  /* PAD, src/rt_ops_f32.c:503-508 */
void orc_expf_n(const float *x, float *y, long long n);  /* the C library's expf, elementwise */
/* STEM fp16 out (src/rt_ops_f16.c:167-180) */
void orc_stem_f32to16(const float *img, int H, int W, int k, int s, int Ho, int Wo, const float *w, const float *b, int Kp,
                      int N, int Np, int act, uint16_t *out, int ldo, int opad);
/* SE fp16 in place (src/v24_fast.c:182-234) */
void orc_se_f16(uint16_t *D, int P, int C, const float *chsum, int rd, const float *w1, const float *b1, const float *w2t,
                const float *b2);
void orc_mean_f16(const uint16_t *x, int P, int C, int ld, float *out);  /* src/pc_kern_f16.c:115-121 */
/* GEMV with fp32 (w16 NULL) or fp16 weights (src/gemv.c:13-49) */
void orc_gemv(const float *w32, const uint16_t *w16, const float *b, int N, int K, const float *x, int act, float *out);

/* ---------------------------------------------------------------- dotprod + fp16 family (dot.c) */
void orc_stem3_f32h(const float *img, int H, int W, const float *w, const float *b, uint16_t *out);

void orc_quant_cells_f16(const uint16_t *x, int P, int C, int ld, float eps, int8_t *qa, int Kp, float *sx);
void orc_proto_colmax_c12(const int8_t *qa, int Kp, const float *sx, int P, int K, const int8_t *qw, const float *sw,
                          int Np, float *colmax);

/* ---------------------------------------------------------------- dotprod int8 (qdot.c) */
typedef struct {
  int act;          /* 0 none, 1 SiLU, 2 ReLU (src/kern.h:31) */
  uint16_t *out16;  /* fp16 output, or NULL */
  float *out32;     /* fp32 output, or NULL */
  int ldo, ow, opad;
  const float *res32;  /* fp32 residual rows [M][ldo], or NULL */
} orc_qd_epi;          /* src/kern.h:33-40 */
void orc_qd_wpack(const float *w, const float *bias, int N, int K, int8_t *q, float *scale, float *swsum, float *b);
void orc_qd_params(float mn, float mx, float *scale, float *zp, float *inv);
void orc_qd_quant_rows_f32(const float *x, int ldx, int M, int C, int8_t *a, int lda, int Cp, float *rq);
void orc_qd_quant_rows_f16(const uint16_t *x, int ldx, int M, int C, const uint16_t *gate, int8_t *a, int lda, int Cp,
                           float *rq);
float orc_exp2_p5(float t);
float orc_silu_f32_a(float x);
float orc_log2_dot(float x);
void orc_qd_gemm(const int8_t *a, int lda, const float *rq, int per_tensor, int M, int N, int Kp, const int8_t *q,
                 const float *scale, const float *swsum, const float *b, const orc_qd_epi *e);
void orc_qpw(const void *x, int in_f16, int ldx, int M, int K, const uint16_t *gate, int8_t *a8, float *rq, int N,
             const int8_t *q, const float *scale, const float *swsum, const float *b, const orc_qd_epi *e);
void orc_qd_quant_tensor_pad(const float *x, int H, int W, int C, int8_t *out, float *rq);
void orc_qconv3(const float *x, int H, int W, int C, int K, int s, int pt, int pl, int Ho, int Wo, const int8_t *q,
                const float *scale, const float *swsum, const float *b, int8_t *xp, int8_t *col, uint16_t *out);
void orc_se_gate16(float *chsum, int C, int rd, int P, const float *w1, const float *b1, const float *w2,
                   const float *b2, uint16_t *gate);
void orc_gem_a(const float *F, int M, int C, float eps, float p, float *e);
/* the C library's powf, elementwise */
void orc_powf_vec(const float *x, const float *y, float *z, long long n);
void orc_heads_s8(const float *F, const float *emb, int H, int W, int C, int hid, int nc, const int8_t *const *wq,
                  const float *const *sc, const float *const *ss, const float *const *bb, float *logits, float *work);

#ifdef __cplusplus
}
#endif
/* ---------------------------------------------------------------- sub-steps exposed for their order tests */
/* fft_dit_x4 (src/fft_tab.h:25-80) on one lane */
void orc_fft_dit(float *re, float *im, int M, const float *twr, const float *twi);
/* v24k32_se_fc1 (src/v24_f32.c:164-179); h16: fp16-held weights (SE_GATE16, src/rt_ops_dot.c:381-420) */
void orc_se_fc1(const float *mean, int C, int rd, const float *w1, int h16, const float *b1, float *s1);
/* HEADS_S8's pooling and attention pooling of one head (src/rt_ops_dot.c:531-570) */
void orc_heads_pool(const float *F, int H, int W, int C, int i, float *s, float *pooled);
void orc_heads_softmax(float *att, const float *cla, int L, int nc, int ncp, float *logits);

#endif
