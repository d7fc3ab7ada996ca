/* libbnneon_hip kernel-level C ABI: the quantized conv / GEMM hot path of libbnneon on MI355X (gfx950).
 *
 * These entry points take DEVICE pointers (HBM) and a HIP stream (NULL = the default stream) and run one kernel
 * family over B windows at once. Every buffer argument names the first window; the window w of a buffer starts
 * `*_ws` ELEMENTS after it (its per-window stride). Each entry point replaces the reference function cited in its
 * comment (paths relative to the reference checkout) and computes, per window, exactly what that function computes
 * (bit-identical for the int8 paths).
 *
 * Return value: 0 on success; -1 with bnh_last_error() (thread-local, <= 511 bytes) describing the failure.
 * Shapes are checked on the host before any launch; nothing here allocates device memory except the *_new
 * constructors and bnh_malloc.
 */
#ifndef BNNEON_HIP_H
#define BNNEON_HIP_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ device plumbing (for hosts without a HIP
 * runtime of their own: ctypes, cgo). No counterpart in the reference, which has no device memory. */
const char *bnh_last_error(void);
int bnh_device_count(void);
void *bnh_malloc(size_t bytes);                                   /* NULL on failure */
int bnh_free(void *p);
int bnh_memcpy_h2d(void *dst, const void *src, size_t bytes);     /* synchronous */
int bnh_memcpy_d2h(void *dst, const void *src, size_t bytes);     /* synchronous */
int bnh_memset(void *dst, int value, size_t bytes);               /* synchronous */
void *bnh_stream_new(void);
int bnh_stream_free(void *stream);
int bnh_stream_sync(void *stream);
void *bnh_event_new(void);
int bnh_event_free(void *ev);
int bnh_event_record(void *ev, void *stream);
float bnh_event_ms(void *start, void *stop);                      /* after both completed; < 0 on error */
/* a plain streaming device-to-device copy (16-byte aligned, bytes % 16 == 0): the bandwidth and HBM-counter
 * calibration reference of the benchmarks */
int bnh_copy(void *dst, const void *src, size_t bytes, void *stream);

/* ------------------------------------------------------------------ scalar numerics checks
 * y[i] = f(x[i]) on the device for n elements, f = 0: FRECPE, 1: the fp32 SiLU of the epilogues
 * (src/gemm_f32.h:102-118) in the form the kernels use (FRECPE's estimate from an LDS table), 2: ReLU (vmaxq_f32
 * with 0), 3: the same SiLU without the table. Used to pin the device numerics against the oracle. */
int bnh_eval_f32(int f, const float *x, float *y, long long n, void *stream);
/* y[i] = the Q31 requantisation of the int8 GEMM / depthwise below applied to acc[i] with mult[i], shift[i] (0..31),
 * zy, clamp [lo, hi]: pins the device fixed-point arithmetic against the oracle. Both device forms (the general one
 * and the one-rounding form for shift 1..31) are evaluated; where they disagree y[i] = INT32_MIN. */
int bnh_eval_requant(const int32_t *acc, const int32_t *mult, const int32_t *shift, int zy, int lo, int hi, int32_t *y,
                     long long n, void *stream);

/* ------------------------------------------------------------------ int8 GEMM weights (PW_S8 / GEMV_S8)
 * Built from the package tensors of one int8 GEMM (python/bnneon/compiler/lower.py:883-914, s8_tensors; validated
 * by s8_view, src/rt_ops_s8n.c:13-25): host arrays w int8 [Np/4][Kp/16][4][16], sw f32 [>= Np], colsum i32 [>= Np],
 * b f32 [>= Np]. The weights are repacked once into the MFMA operand order and kept in HBM. */
typedef struct bnh_s8w bnh_s8w;
bnh_s8w *bnh_s8w_new(int N, int K, int Kp, int Np, const int8_t *w, const float *sw, const int32_t *colsum,
                     const float *b);
void bnh_s8w_free(bnh_s8w *W);

/* the fp32 epilogue of the int8 GEMM (epi32, src/gemm_f32.h:15-24), with per-window strides */
typedef struct {
  int act;               /* 0 none, 1 SiLU, 2 ReLU */
  float *out;            /* pixel m at row m (opad 0) or ((m/ow)+opad)*(ow+2opad) + m%ow + opad */
  long long out_ws;
  int ldo, ow, opad;
  const float *res;      /* optional residual (NULL), added after the activation */
  long long res_ws;
  int ldr, rpad, rw;
} bnh_epi32;

/* s8n_quant_rows / s8n_quant_rows_gate (src/gemm_s8n.c:15-63; declared src/gemm_s8n.h:15-17): rows [0, M) of
 * each window -> q int8 [M][Kp] (pad k = the zero point), sa f32 [M], za i32 [M]. gate (or NULL): f32 [K] per
 * window (stride gate_ws), K % 4 == 0 and K <= 4096 as the reference requires. */
int bnh_s8n_quant_rows(const float *x, long long x_ws, int ld, int M, int K, int Kp, const float *gate,
                       long long gate_ws, int8_t *q, long long q_ws, float *sa, long long sa_ws, int32_t *za,
                       long long za_ws, int B, void *stream);
/* s8n_gemm_range over every row and panel (src/gemm_s8n.c:176-190; src/gemm_s8n.h:21-22): out rows [0, M) x
 * channels [0, Np) = act(dequant(q . W) + b) (+ residual), stored by the epi32 rules */
int bnh_s8n_gemm(const int8_t *q, long long q_ws, const float *sa, long long sa_ws, const int32_t *za, long long za_ws,
                 int M, int B, const bnh_s8w *W, const bnh_epi32 *e, void *stream);
/* the PW_S8 op run (pw8_run, src/rt_ops_s8n.c:119-134): zero the output halo when opad (H = M / ow), quantize
 * (gated when gate != NULL) and multiply, for B windows */
int bnh_pw_s8(const float *in, long long in_ws, int lda, int M, const float *gate, long long gate_ws, int8_t *q,
              long long q_ws, float *sa, long long sa_ws, int32_t *za, long long za_ws, int B, const bnh_s8w *W,
              const bnh_epi32 *e, void *stream);
/* bnh_pw_s8 without a workspace and without any device allocation. No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, serving loops or harnesses that forbid hipMalloc).
 * The quantized rows, scales and zero points live in a library-owned static device array of 64 MiB per device:
 * B * M * Kp + 8 * B * M bytes (each part rounded up to 256) must fit, else -1 with a message and nothing launched.
 * Calls on one device share that array, so calls that overlap on one device (other streams, other threads) race;
 * each call rewrites every part of it that it reads. Same outputs as bnh_pw_s8, bit for bit. */
int bnh_pw_s8_static(const float *in, long long in_ws, int lda, int M, const float *gate, long long gate_ws, int B,
                     const bnh_s8w *W, const bnh_epi32 *e, void *stream);

/* ------------------------------------------------------------------ int8 prototype head (PROTO_S8)
 * Prototypes from the package tensors of PROTO_S8 (src/rt_ops_s8n.c:212-236): qw int8 [Np/4][Kp/16][4][16] and sw
 * f32 [>= Np], repacked once into MFMA operand rows in HBM. */
typedef struct bnh_s8p bnh_s8p;
bnh_s8p *bnh_s8p_new(int Np, int Kp, const int8_t *qw, const float *sw);
void bnh_s8p_free(bnh_s8p *W);
/* pc_quant_cells_f32 (src/proto_s8n.c:28-51; declared src/pc_kern.h:60): cells x [P][ld] (C channels, C % 8 == 0)
 * -> qa int8 [P][Kp] in [-127, 127] (zeros past C) and sx f32 [P], the scales of the L2-normalised cells */
int bnh_quant_cells(const float *x, long long x_ws, int P, int C, int ld, float eps, int8_t *qa, long long qa_ws,
                    int Kp, float *sx, long long sx_ws, int B, void *stream);
/* pc_quant_cells_f16 (src/pc_proto_s8.c:14-45): fp16 cells; the codes saturate to [-128, 127] (no floor at -127) */
int bnh_quant_cells_f16(const uint16_t *x, long long x_ws, int P, int C, int ld, float eps, int8_t *qa,
                        long long qa_ws, int Kp, float *sx, long long sx_ws, int B, void *stream);
/* the dotprod head's prototypes (PROTO variant 2, src/rt_ops_f16.c:252-281): qw int8 [Np/12][K/4][12][4], sw f32
 * [Np], K % 4 == 0, repacked as bnh_s8p_new's with Kp = K rounded up to 16 */
bnh_s8p *bnh_s8p_new_c12(int Np, int K, const int8_t *qw, const float *sw);
/* pc_proto_colmax_s8n over every panel (src/proto_s8n.c:139-164; src/pc_kern.h:64-65): colmax f32 [Np] per window,
 * the maximum over the window's P cells of (float)(qa . qw) * sx, times sw */
int bnh_proto_colmax(const int8_t *qa, long long qa_ws, const float *sx, long long sx_ws, int P, const bnh_s8p *W,
                     float *colmax, long long cm_ws, int B, void *stream);
/* pc_proto_logits (src/pc_kern_f32.c:364-374; src/pc_kern.h:69): logits f32 [nc] per window from colmax and the
 * class tensors clsw f32 [nc][ppc], clsb f32 [nc] (device). A window with a non-finite logit gets
 * win_fail[w] = fail_code (when still 0; win_fail may be NULL) -- the reference's return value -2. */
int bnh_proto_logits(const float *colmax, long long cm_ws, const float *clsw, const float *clsb, int nc, int ppc,
                     float *logits, long long lg_ws, int B, int *win_fail, int fail_code, void *stream);

/* ------------------------------------------------------------------ fp32 / fp16 prototype heads
 * PROTO variant 0 (src/rt_ops_f32.c:548-570), PROTO_F32H (src/rt_ops_f32.c:572-591) and PROTO variant 1
 * (src/rt_ops_f16.c:227-250). Prototypes from the package tensor, K % 8 == 0 and Np % 8 == 0:
 *   kind 0: fp32 panels [Np/8][K][8] (fpack, Kp = K), kind 1: fp16 panels [Np/8][K][8] (PROTO_F32H),
 *   kind 2: fp16 panels [Np/16][K][16] then a tail panel [K][8] when Np % 16 == 8 (hpack, Kp = K);
 * repacked once into k-major rows in HBM. */
typedef struct bnh_fproto bnh_fproto;
bnh_fproto *bnh_fproto_new(int kind, int Np, int K, const void *w);
void bnh_fproto_free(bnh_fproto *W);
/* pc_l2norm_f32 (src/pc_kern_f32.c:350-362) or, f16 != 0, pc_l2norm_f16 (src/pc_kern_f16.c:123-140): cells x [P][ld]
 * (fp32, or fp16 bit patterns) -> a [P][C] of the same type, each cell divided by sqrtf(sum of squares) + eps */
int bnh_l2norm_cells(const void *x, long long x_ws, int P, int C, int ld, float eps, int f16, void *a, long long a_ws,
                     int B, void *stream);
/* gemm_f32_colmax (src/gemm_f32.c:443-460), pc_proto_colmax_f32h (src/pc_kern_f32.c:378-407) or gemm_f16_colmax
 * (src/gemm_f16.c:210-253) by W's kind: colmax f32 [Np] per window, the maximum over the window's P cells a [P][K]
 * (fp32; fp16 for kind 2; 16-byte aligned) of their products with each prototype, summed as the reference does */
int bnh_fproto_colmax(const void *a, long long a_ws, int P, const bnh_fproto *W, float *colmax, long long cm_ws, int B,
                      void *stream);

/* ------------------------------------------------------------------ int8 GEMM with Q31 requantisation
 * No counterpart in the reference (whose int8 GEMM dequantises to fp32): the TFLite-style static int8 pointwise
 * convolution, NCHW. Per window: x int8 [K][M] (pixels contiguous), out int8 [N][M];
 *   acc = sum_k w[n][k] (x[k][m] - zx) + bias[n];
 *   out = clamp(RoundingDivideByPOT(SaturatingRoundingDoublingHighMul(acc, mult[n]), shift[n]) + zy, lo, hi).
 * Weights are uploaded once (host w int8 [N][K], bias / mult / shift int32 [N]). */
typedef struct bnh_q8w bnh_q8w;
bnh_q8w *bnh_q8w_new(int N, int K, const int8_t *w, const int32_t *bias, const int32_t *mult, const int32_t *shift,
                     int zx, int zy, int lo, int hi);
void bnh_q8w_free(bnh_q8w *W);
int bnh_gemm_s8_requant(const bnh_q8w *W, const int8_t *x, long long x_ws, int M, int B, int8_t *out,
                        long long out_ws, void *stream);

/* ------------------------------------------------------------------ fp16 GEMM (PW f16)
 * Weights from the package tensors of an fp16 GEMM (hp_pack, src/gemm_f16.c:18-40; validated as hpack_view,
 * src/rt_ops_f16.c:14-27): w fp16 [Np/16][Kp][16] then, if Np % 16, a tail panel [Kp][8]; b32 f32 [>= Np];
 * b16 fp16 [>= Np], the package's fp16 bias (NULL: b32 rounded to nearest even). Repacked once into channel rows
 * in HBM. */
typedef struct bnh_h16w bnh_h16w;
bnh_h16w *bnh_h16w_new(int N, int K, int Kp, int Np, const uint16_t *w, const float *b32, const uint16_t *b16);
void bnh_h16w_free(bnh_h16w *W);
/* the fp16 epilogue (epi16, src/gemm_f16.h:19-27, without the pooled form), per-window strides in elements */
typedef struct {
  int act;               /* 0 none, 1 SiLU (the fp16 LUT form), 2 ReLU */
  uint16_t *out;         /* fp16; pixel m at row m (opad 0) or ((m/ow)+opad)*(ow+2opad) + m%ow + opad */
  long long out_ws;
  int ldo, ow, opad;
  const uint16_t *res;   /* optional fp16 residual [M][ldr], added after the activation */
  long long res_ws;
  int ldr;
} bnh_epi16;
/* gemm_f16 (src/gemm_f16.c:124-171; the PW f16 op run, src/rt_ops_f16.c:65-81): out rows [0, M) x channels [0, Np)
 * of act(A . W^T + b) (+ res) for B windows of fp16 rows A [M][lda] (lda >= Kp, lda % 8 == 0; zero-haloed output
 * zeroed when opad). Bit-identical to the reference: fp16 FMA chains over its K blocks (packed fp16 FMAs on the
 * VALU), fp32 sums across blocks, its bias and epilogue. */
int bnh_gemm_f16(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W, const bnh_epi16 *e,
                 void *stream);
/* bnh_gemm_f16 without its halo zeroing, for callers whose output halo is already zero (the runtime's buffers that
 * own their arena slot keep the zero halo written when the arena was cleared) */
int bnh_gemm_f16_body(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W, const bnh_epi16 *e,
                      void *stream);
/* bnh_gemm_f16_body with a workspace ws (16-byte aligned) of at least bnh_gemm_f16_ws_bytes(M, B, W) bytes: when the
 * product has several K blocks and too few rows to fill the GPU, every K block runs as its own set of blocks and a
 * second kernel sums their fp16 results in fp32 in the reference's block order (the same bits). ws NULL or too small:
 * the one-kernel form. */
size_t bnh_gemm_f16_ws_bytes(int M, int B, const bnh_h16w *W);
int bnh_gemm_f16_ws(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W, const bnh_epi16 *e,
                    void *ws, size_t ws_bytes, void *stream);
/* the same product of the gated rows A x gh: A's column k multiplied by the window's fp16 gate gh[k] (gh [B][gh_ws]
 * fp16, gh_ws >= Kp) as it is loaded. The fp16 SE (src/rt_ops_f32.c:256-327) scales A in place by the same fp16
 * products before the reference's 1x1 conv reads it; here the scaling happens in the GEMM's A-load and A is left as
 * it was (no reference counterpart as an entry point). */
int bnh_gemm_f16_gated_ws(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W,
                          const bnh_epi16 *e, const uint16_t *gh, long long gh_ws, void *ws, size_t ws_bytes,
                          void *stream);
/* the same product on fp16 MFMA with fp32 accumulation over the whole K (no reference counterpart: a faster form
 * for callers that accept the fp16 accumulation error bound of the reference instead of its exact bits) */
int bnh_gemm_f16_mfma(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W, const bnh_epi16 *e,
                      void *stream);
/* the same with A's columns multiplied by the window's fp16 gates gh [>= Kp] (stride gh_ws) as they are loaded (no
 * reference counterpart: the MFMA form of bnh_gemm_f16_gated_ws, an fp16 SE's scaling fused into its projection) */
int bnh_gemm_f16_mfma_gated(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W,
                            const bnh_epi16 *e, const uint16_t *gh, long long gh_ws, void *stream);

/* ------------------------------------------------------------------ fp16 Winograd F(2x2, 3x3) convolution
 * The Winograd / fp16 GEMM path (src/wino_s0.c:1-165 for the transforms, src/wino.c for the tiling): a 3 x 3,
 * stride 1, pad 1 convolution of C <= 64 input channels (C % 4 == 0) into K <= 64 output channels. Weights OHWI fp32
 * [K][3][3][C] and bias [K] are transformed once (U = G g G^T in fp32, rounded to fp16, as wino_s0_pack). Per window:
 * x fp16 zero-haloed [H+2][W+2][ldx] (H, W even); out fp16 [H][W][ldo] (opad 0) or zero-haloed [H+2][W+2][ldo]
 * (opad 1); optional fp16 residual added last, [H][W][ldr] (rpad 0) or zero-haloed [H+2][W+2][ldr] (rpad 1: the
 * CONV3C24 form, src/rt_ops_dot.c:63-107, whose residual is its own haloed input). V = B^T d B in fp16 (wino_s0.c's order), the 16
 * position GEMMs on fp16 MFMA with fp32 accumulation, y = A^T M A + b and the activation (0 none, 1 the fp32 SiLU,
 * 2 ReLU) in fp32, one rounding to fp16. Within the fp16 Winograd error bound of a direct convolution (the
 * parity tests state it), not bit-identical to the reference's fp16 chains. */
typedef struct bnh_wino16 bnh_wino16;
bnh_wino16 *bnh_wino16_new(int C, int K, const float *w, const float *bias);
void bnh_wino16_free(bnh_wino16 *P);
int bnh_wino_f16(const uint16_t *x, long long x_ws, int H, int W, int ldx, const bnh_wino16 *P, int act, uint16_t *out,
                 long long o_ws, int ldo, int opad, const uint16_t *res, long long r_ws, int ldr, int rpad, int B,
                 void *stream);

/* ------------------------------------------------------------------ int8 Winograd F(2x2, 3x3) (WINO_S8)
 * libbnneon's int8 Winograd for 3 x 3 stride-1 pad-1 convolutions (wino_pack / wino_f23_tiles, src/wino.c:26-227;
 * the WINO_S8 op, src/rt_ops_dot.c:130-170), bit-identical: weights OHWI fp32 [K][3][3][C] and bias [K] are packed
 * once (U = G g G^T quantised per output channel); per window x f32 [H][W][C] (rows, ld C) -> out fp16 [H][W][K]
 * (ld K) = SiLU(conv + b) with per-tile asymmetric int8 activations. C % 8 == 0, K % 16 == 0, both <= 2048. work:
 * device scratch of at least bnh_wino8_work_bytes(H, W, C, B) bytes (the quantised tiles and their scales). */
typedef struct bnh_w8w bnh_w8w;
bnh_w8w *bnh_wino8_new(int C, int K, const float *w, const float *bias);
void bnh_wino8_free(bnh_w8w *P);
size_t bnh_wino8_work_bytes(int H, int W, int C, int B);
int bnh_wino_s8(const float *x, long long x_ws, int H, int W, const bnh_w8w *P, uint16_t *out, long long o_ws, int B,
                void *work, size_t work_bytes, void *stream);

/* ------------------------------------------------------------------ depthwise convolutions
 * NHWC, weights [k*k][C] (tap-major), per-window strides in elements. xp is the zero-haloed input of the reference's
 * buffers: [H + 2h][W + 2h][C], h = (k - 1) / 2 (1 for the DW3 forms); output pixel (oy, ox) reads the k x k taps
 * from halo row oy*s - pt + h, column ox*s - pl + h. chsum (optional, fp32 [C] per window) receives the per-channel
 * sum of the outputs in the reference's order (the SE block's mean input). Every result is bit-identical to the
 * reference's NEON kernel. act: 0 none, 1 SiLU. */
/* DWK fp32, k in {1, 3, 5, 7}, s in {1, 2}: replaces dwk_f32_run (src/pc_kern_f32.c:163-334) */
int bnh_dwk_f32(const float *xp, long long x_ws, int H, int W, int C, int k, int s, int pt, int pl, const float *w,
                const float *b, int act, float *out, long long o_ws, int Ho, int Wo, float *chsum, long long cs_ws,
                int B, void *stream);
/* DW3 fp32 (3x3, pads 1, SiLU): replaces dw3_f32 / dw3s2_f32 (src/gemm_f32.c:213-441) */
int bnh_dw3_f32(const float *xp, long long x_ws, int H, int W, int C, int s, const float *w, const float *b, float *out,
                long long o_ws, int Ho, int Wo, float *chsum, long long cs_ws, int B, void *stream);
/* An int8 1x1 expansion fused into the fp32 depthwise conv that is its only reader: no reference counterpart (the
 * reference runs PW_S8 into a zero-haloed buffer, then DW3 / DWK over it; src/rt_ops_s8n.c:92-134 and
 * src/rt_ops_f32.c:216-232, 435-458). From the PW_S8 rows already quantized by bnh_s8n_quant_rows (q, sa, za over
 * M = H W pixels) and W's C = W->Np channels with activation pact, it writes exactly the outputs (and per-channel
 * sums) bnh_s8n_gemm into a halo-(k-1)/2 buffer followed by bnh_dw3_f32 (form 2: k 3, pads 1) or bnh_dwk_f32
 * (form 0, activation dact) would write, without the expanded tensor. C % 16 == 0, k in {3, 5}. */
int bnh_pwdw_f32(const int8_t *q, long long q_ws, const float *sa, long long sa_ws, const int32_t *za, long long za_ws,
                 int H, int W, const bnh_s8w *Wt, int pact, int k, int s, int pt, int pl, int form, const float *w,
                 const float *b, int dact, float *out, long long o_ws, int Ho, int Wo, float *chsum, long long cs_ws,
                 int B, void *stream);
/* DWK fp16 (values as fp16 bit patterns): replaces dwk_f16_run (src/pc_kern_f16.c:16-96) */
int bnh_dwk_f16(const uint16_t *xp, long long x_ws, int H, int W, int C, int k, int s, int pt, int pl,
                const uint16_t *w, const uint16_t *b, int act, uint16_t *out, long long o_ws, int Ho, int Wo,
                float *chsum, long long cs_ws, int B, void *stream);
/* DW3 fp16 (3x3, SiLU, pads pt / pl in {0, 1}): replaces dw3_f16 (src/kern_f16.c:83-155) */
int bnh_dw3_f16(const uint16_t *xp, long long x_ws, int H, int W, int C, int s, int pt, int pl, const uint16_t *w,
                const uint16_t *b, uint16_t *out, long long o_ws, int Ho, int Wo, float *chsum, long long cs_ws, int B,
                void *stream);
/* int8 depthwise: no counterpart in the reference (its depthwise layers are fp32 / fp16); the static int8 form of
 * the same layer. x int8 [H][W][C] unpadded (C % 4 == 0), taps outside the image skipped (a zero-point pad):
 *   acc = bias[c] + sum_taps w[t][c] (x - zx);  y = clamp(RDBYPOT(SRDHM(acc, mult[c]), shift[c]) + zy, lo, hi);
 *   out = lut ? lut[y + 128] : y   (lut: an int8 -> int8 activation table, e.g. SiLU)
 * zx is the input's int8 zero point (-128..127); x, w and out 4-byte aligned. */
int bnh_dw_s8(const int8_t *x, long long x_ws, int H, int W, int C, int k, int s, int pt, int pl, const int8_t *w,
              const int32_t *bias, const int32_t *mult, const int32_t *shift, int zx, int zy, int lo, int hi,
              const int8_t *lut, int8_t *out, long long o_ws, int Ho, int Wo, int B, void *stream);

/* ------------------------------------------------------------------ fp32 ops around the int8 GEMMs
 * The fp32 registry ops of the int8 Perch-family plan, bit-identical to the reference's kernels. Per-window strides in
 * elements; B windows per launch. */
/* FE_LOGMEL: replaces pc_logmel_new / pc_logmel_run (src/pc_kern_f32.c:28-149): pcm [nsamp] -> spec f32
 * [nfr][nmel], nfr = (nsamp + 2 pad - frame) / hop + 1; window [frame]; mel dense [nmel][nfft/2 + 1] (kept sparse);
 * spec = ln(max(mel . |FFT|, floor)) * scale with the reference's radix-2 FFT and log2 polynomial. nfft a power of
 * two in 16..2048, frame <= nfft, nmel <= 512 (the reference's limits). */
typedef struct bnh_logmel bnh_logmel;
bnh_logmel *bnh_logmel_new(int nsamp, int frame, int hop, int pad, int nfft, int nmel, const float *window,
                           const float *mel, float floor_, float scale);
void bnh_logmel_free(bnh_logmel *F);
int bnh_logmel_frames(const bnh_logmel *F);
int bnh_logmel_run(const bnh_logmel *F, const float *pcm, long long p_ws, float *spec, long long s_ws, int B, void *stream);
/* fp32 GEMM of the PW op: replaces gemm_f32 / gemm_f32_range_gate (src/gemm_f32.c:141-197; called by pw_run,
 * src/rt_ops_f32.c:198-207): A f32 [M][lda] per window (lda >= Kp; rows < M read), gate (or NULL) f32 [Kp] per window
 * scaling A[m][k] first, w the package's fp32 panels [Np/8][Kp][8] (Kp % 4 == 0, 16-byte aligned), bias [Np] ->
 * e->out rows [0, M) x channels [0, Np) = act(A . W + b) (+ residual), stored by the epi32 rules. Every output is the
 * reference's FMA chain over k < Kp, bit for bit. */
int bnh_gemm_f32(const float *A, long long a_ws, int lda, int M, const float *gate, long long g_ws, const float *w,
                 const float *bias, int Kp, int Np, const bnh_epi32 *e, int B, void *stream);
/* STEM: replaces stem_run (src/rt_ops_f32.c:416-425; pc_im2col1 + gemm_f32): a 1-channel image [H][W], VALID k x k
 * stride s -> out [Ho][Wo][ldo] (opad: zero-haloed [Ho+2opad][Wo+2opad][ldo]) = act(conv + b), channels < Np stored;
 * w the package's fp32 panels [Np/8][Kp][8] (Kp >= k*k, Kp % 4 == 0; 16-byte aligned), bias [Np]. act 0/1/2. */
int bnh_stem_f32(const float *img, long long i_ws, int H, int W, int k, int s, int Ho, int Wo, const float *w,
                 const float *bias, int Kp, int Np, int act, float *out, long long o_ws, int ldo, int opad, int B,
                 void *stream);
/* SE_GATE / SE: replaces seg_run and se_run (src/rt_ops_f32.c:297-324; v24k32_se_fc1 / v24k32_se, src/v24_f32.c:
 * 164-210): from the channel sums chsum [C] of P pixels, gate [C] = sigmoid(w2 silu(w1 mean + b1) + b2) (w1 [rd][C],
 * b1 [rd], w2t [rd][C], b2 [C]; silu by the C library's expf, as the reference). gate (or NULL) receives it; D (or
 * NULL) [P][C] is multiplied by it in place (with both and C % 8 == 0 by a second kernel over every window's
 * pixels, the fast form). work (or NULL): a workspace of B x rd floats; with it and gate the two FCs run as
 * kernels over all windows (the fast form), without it one kernel per group of windows computes them.
 * C % 4 == 0, C <= 4096, rd <= 512. */
int bnh_se_f32(const float *chsum, long long c_ws, int C, int rd, int P, const float *w1, const float *b1,
               const float *w2t, const float *b2, float *gate, long long g_ws, float *work, float *D, long long d_ws,
               int B, void *stream);
/* STEM of the fp16 path: replaces stem_run (src/rt_ops_f16.c:167-180): the fp32 stem above, then channels < N
 * rounded to fp16 into out fp16 [Ho+2opad][Wo+2opad][ldo] (halo zeroed; channels N..ldo untouched) */
int bnh_stem_f32to16(const float *img, long long i_ws, int H, int W, int k, int s, int Ho, int Wo, const float *w,
                     const float *bias, int Kp, int N, int Np, int act, uint16_t *out, long long o_ws, int ldo, int opad,
                     int B, void *stream);
/* SE of the fp16 path: replaces se_run (src/rt_ops_f16.c:125-137; v24k16_se, src/v24_fast.c:182-234): the gate as
 * bnh_se_f32 computes it but with a dividing sigmoid, rounded to fp16; D fp16 [P][C] multiplied by it in fp16.
 * gate: optional workspace fp32 [B][g_ws >= C] that receives the (unrounded) gates; with it and C % 8 == 0 the
 * scaling runs as its own kernel over every window's pixels (the fast form); NULL computes and applies the gates in
 * one kernel per group of windows. work: as for bnh_se_f32. */
int bnh_se_f16(const float *chsum, long long c_ws, int C, int rd, int P, const float *w1, const float *b1,
               const float *w2t, const float *b2, float *gate, long long g_ws, float *work, uint16_t *D,
               long long d_ws, int B, void *stream);
/* the fp16 SE's gates alone (fp32 into gate, their fp16 roundings, the factors the scaling multiplies by, into gh
 * [B][gh_ws]), D untouched: for bnh_gemm_f16_gated_ws (C % 8 == 0; no reference counterpart as an entry point) */
int bnh_se_gate_f16(const float *chsum, long long c_ws, int C, int rd, int P, const float *w1, const float *b1,
                    const float *w2t, const float *b2, float *gate, long long g_ws, float *work, uint16_t *gh,
                    long long gh_ws, int B, void *stream);
/* MEAN of fp16 rows: replaces pc_mean_f16 (src/pc_kern_f16.c:115-121) */
int bnh_mean_f16(const uint16_t *x, long long x_ws, int P, int C, int ld, float *out, long long o_ws, int B,
                 void *stream);
/* GEMV: replaces bnn_gemv_f32 / bnn_gemv_h16 (src/gemv.c:13-49): out [N] = act(b + W x), W [N][K] fp32 (w16 = 0) or
 * fp16 (w16 = 1) weights, fp32 arithmetic in the reference's lane order; act 0 or 2 (ReLU) */
int bnh_gemv(const void *w, int w16, const float *bias, int N, int K, const float *x, long long x_ws, int act,
             float *out, long long o_ws, int B, void *stream);
/* MEAN: replaces pc_mean_f32 (src/pc_kern_f32.c:342-348): out [C] = (sum over P rows of x [P][ld]) / P */
int bnh_mean_f32(const float *x, long long x_ws, int P, int C, int ld, float *out, long long o_ws, int B,
                 void *stream);
/* STEM3: replaces stem3_run (src/rt_ops_dot.c:46-61; stem_conv_f32_h, src/kern_f16.c:15-71): img f32 [H][W][3] ->
 * out fp16 zero-haloed [(H+1)/2 + 2][(W+1)/2 + 2][24] (the halo is left as it is) = the table SiLU of the fp16 rounding
 * of the 3 x 3 stride-2 conv (taps past the bottom / right edge skipped) + b; w OHWI fp32 [24][3][3][3], b [24]. out
 * 16-byte aligned. Bit-identical. */
int bnh_stem3_f16(const float *img, long long i_ws, int H, int W, const float *w, const float *b, uint16_t *out,
                  long long o_ws, int B, void *stream);
/* UNPAD: replaces unpad_run (src/rt_ops_dot.c:109-128): the interior of a zero-haloed fp16 buffer [H+2][W+2][C]
 * widened to fp32 rows [H][W][C] (W C % 4 == 0; out 16-byte aligned) */
int bnh_unpad_f16(const uint16_t *x, long long x_ws, int H, int W, int C, float *out, long long o_ws, int B,
                  void *stream);
/* PAD: replaces pad_run (src/rt_ops_f32.c:503-508, src/rt_ops_f16.c:204-210): rows [H][W][ld] -> zero-haloed
 * [H+2h][W+2h][C], elements of esz (4 or 2) bytes */
int bnh_pad(const void *x, long long x_ws, int H, int W, int C, int ld, int h, int esz, void *xp, long long p_ws, int B,
            void *stream);
/* rt_zero_halo (src/rt_pkg.c:194-203) on every window: zeroes the halo of [H+2h][W+2h][C], elements of esz bytes */
int bnh_zero_halo(void *xp, long long ws, int H, int W, int C, int h, int esz, int B, void *stream);
/* test hook: y = expf(x) as the C library computes it (glibc's table method), elementwise on the device */
int bnh_eval_expf(const float *x, float *y, long long n, void *stream);
/* test hook: z = powf(x, y) as the C library computes it (glibc's table method), elementwise on the device */
int bnh_eval_powf(const float *x, const float *y, float *z, long long n, void *stream);

/* ------------------------------------------------------------------ dotprod int8 family (QPW, QCONV3, HEADS_S8)
 * libbnneon's int8 SDOT arithmetic (src/gemm_s8.c), bit-identical: activations quantised per row (or per tensor) to
 * [-128, 127] with scale s and float zero point zp (rq = {s, zp} pairs), weights per channel to [-127, 127]; int32
 * sums, then v = (b + (acc sw) s) + swsum (s zp), both sums fused; fp16 out (act 0 / 1: the table SiLU) or fp32 out
 * (act 0 / 1 / 2: silu_f32_a / ReLU, then + res). Inputs with NaNs are outside what the parity tests cover. */
typedef struct bnh_qdw bnh_qdw;
/* qw_pack (src/gemm_s8.c:10-35): w fp32 [N][K], bias [N] (or NULL); Np >= N, Np % 16 == 0: channels past N are zero
 * rows (pack_padded, src/rt_ops_dot.c:467-473) */
bnh_qdw *bnh_qdw_new(const float *w, const float *bias, int N, int K, int Np);
void bnh_qdw_free(bnh_qdw *W);
int bnh_qdw_shape(const bnh_qdw *W, int *N, int *K, int *Kp, int *Np);
/* quant_rows_f32 / quant_rows_f16 (src/gemm_s8.c:306-371): x rows [M][ldx] (fp32, or fp16 when in_f16, optionally
 * multiplied channel-wise by the fp16 gate [K]) -> a int8 [M][Kp] (Kp = K rounded up to 16, zero past K, a and a_ws
 * 4-byte aligned), rq fp32 [M][2] */
int bnh_qd_quant_rows(const void *x, int in_f16, long long x_ws, int ldx, int M, int K, const uint16_t *gate,
                      long long g_ws, int8_t *a, long long a_ws, float *rq, long long rq_ws, int B, void *stream);
typedef struct {
  int act;          /* 0 none, 1 SiLU, 2 ReLU (fp32 out only) */
  int out_f16;      /* 1: out is fp16, 0: fp32 */
  void *out;        /* rows [M][ldo], or zero-haloed (opad 1, image width ow) rows */
  long long out_ws; /* elements */
  int ldo, ow, opad;
  const float *res; /* fp32 out only: residual rows [M][ldo] (no halo), or NULL */
  long long res_ws;
} bnh_qd_epi;       /* epi (src/kern.h:33-40) */
/* gemm_s8 (src/gemm_s8.c:153-278): a int8 rows [M][lda] (16-byte aligned), rq per row [M][2] (per_tensor: one pair per
 * window) -> the epilogue e over W->Np channels */
int bnh_qd_gemm(const int8_t *a, long long a_ws, int lda, const float *rq, long long rq_ws, int per_tensor, int M,
                const bnh_qdw *W, const bnh_qd_epi *e, int B, void *stream);
/* QCONV3: replaces qconv_run (src/rt_ops_dot.c:177-216): x f32 [H][W][C] -> out fp16 rows [Ho][Wo][Wq->Np] = the table
 * SiLU of the 3 x 3 stride-s conv (TF-same low pads pt, pl) over the per-tensor quantised input; Wq from OHWI weights
 * viewed as [K][9 C]. work: per-window device scratch slots of work_ws >= bnh_qconv3_work_bytes bytes (256-aligned). */
size_t bnh_qconv3_work_bytes(int H, int W, int C);
int bnh_qconv3(const float *x, long long x_ws, int H, int W, int C, int s, int pt, int pl, int Ho, int Wo,
               const bnh_qdw *Wq, uint16_t *out, long long o_ws, int B, void *work, size_t work_ws, void *stream);
/* HEADS_S8: replaces heads_run (src/rt_ops_dot.c:520-572): logits [ncp] = lin(emb) + the two SED heads over F [H*W][C]
 * (per time step the mean over the other axis, max + average pool 3, fc + ReLU, att clipped to [-10, 10] and
 * soft-maxed over time, cla weighted by it). w / b: lin [nc][C], then per head fc [hid][C], att [nc][hid], cla
 * [nc][hid]. a8 / rq: the op's int8 rows ((L + 4) max(C, hid) bytes) and scales (2 (L + 4) floats), L = max(H, W);
 * work: per-window scratch slots of work_ws >= bnh_heads8_work_bytes bytes. */
typedef struct bnh_heads8 bnh_heads8;
bnh_heads8 *bnh_heads8_new(int C, int hid, int nc, const float *const *w, const float *const *b);
void bnh_heads8_free(bnh_heads8 *P);
size_t bnh_heads8_work_bytes(int H, int W, int C, int hid, int nc);
int bnh_heads_s8(const float *F, long long f_ws, const float *emb, long long e_ws, int H, int W, const bnh_heads8 *P,
                 float *logits, long long l_ws, int8_t *a8, long long a8_ws, float *rq, long long rq_ws, int B,
                 void *work, size_t work_ws, void *stream);
/* SE_GATE16: replaces seg_run (src/rt_ops_dot.c:381-420): chsum [C] scaled to means in place (x (1/P)), gate fp16 [C]
 * = sigmoid(fc2(SiLU(fc1(means)))) with fp16-held weights w1 [rd][C], w2 [C][rd] and fp32 arithmetic */
typedef struct bnh_seg16 bnh_seg16;
bnh_seg16 *bnh_seg16_new(int C, int rd, const float *w1, const float *b1, const float *w2, const float *b2);
void bnh_seg16_free(bnh_seg16 *S);
int bnh_se_gate16(float *chsum, long long c_ws, int P, const bnh_seg16 *S, uint16_t *gate, long long g_ws, int B,
                  void *stream);
/* GEM_A: replaces gem_run (src/rt_ops_dot.c:439-465): e [C] = (mean over the M rows of F [M][C] of max(F, eps)^p)^(1/p)
 * with the reference's exp2 / log2 polynomials; the final power is rounded once from double precision, so it may
 * differ from the C library's powf by one unit in the last place */
int bnh_gem_a(const float *F, long long f_ws, int M, int C, float eps, float p, float *e, long long e_ws, int B,
              void *stream);
/* test hook: the family's scalar functions elementwise (f 0 exp2_p5, 1 silu_f32_a, 2 log2_f32, 3 the SE sigmoid) */
int bnh_eval_qd(int f, const float *x, float *y, long long n, void *stream);

#ifdef __cplusplus
}
#endif
#endif
