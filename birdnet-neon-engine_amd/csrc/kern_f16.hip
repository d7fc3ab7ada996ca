// fp16 pointwise-convolution GEMM (libbnneon's gemm_f16, src/gemm_f16.c, the PW op of the fp16 family) on gfx950,
// in two forms:
//  - k_gemm_f16x (bnh_gemm_f16): the reference's own arithmetic, bit-identical: per output an fp16 FMA chain over
//    each K block, fp32 sums across blocks, its bias and epilogue; packed fp16 FMAs on the VALU.
//  - k_gemm_f16 (bnh_gemm_f16_mfma): fp16 MFMA (v_mfma_f32_16x16x32_f16) with fp32 accumulation over the whole K,
//    then the same epilogue (+ bias in fp32, one rounding to fp16, fp16 LUT SiLU or ReLU, fp16 residual add,
//    zero-haloed store); within the fp16 accumulation error bound of the reference's result.
//
// Layouts: A fp16 NHWC rows [M][lda] per window (k contiguous); weights repacked at load from the package's
// [Np/16][Kp][16] + [Kp][8] panels into channel rows [Nt][Kp] (Nt = Np rounded to 128, zero rows past Np); fp32 and
// fp16 biases [Nt].
#include <string.h>

#include "bnh_internal.h"
#include "bnh_num.h"
#include "bnh_f16.h"

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

struct bnh_h16w {
  int N, K, Kp, Np, Nt;
  uint16_t *w;    // [Nt][Kp]
  float *b;       // [Nt] fp32 bias
  uint16_t *b16;  // [Nt] fp16 bias
};

struct Epi16Dev {
  int act;
  uint16_t *out;
  long long out_ws;
  int ldo, ow, opad;
  const uint16_t *res;
  long long res_ws;
  int ldr;
};

// 4 waves as 2 (rows) x 2 (channels); a wave computes 32 rows x 64 channels (2 x 4 MFMA tiles)
__global__ __launch_bounds__(256) void k_gemm_f16(const uint16_t *__restrict__ A, long long a_ws, int lda, int M,
                                                  long long rows, const uint16_t *__restrict__ wt,
                                                  const float *__restrict__ bias, int Kp, int Np, Epi16Dev e) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const long long row0 = (long long)blockIdx.x * 64 + wm * 32;
  const int n0 = blockIdx.y * 128 + wn * 64;
  if (row0 >= rows) return;
  const int kc = (lane >> 4) * 8;  // this lane's k chunk within a 32-wide step (halves)
  const uint16_t *ap[2];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    long long r = row0 + 16 * t + (lane & 15);
    if (r >= rows) r = rows - 1;  // a valid row; its results are not stored
    const int w = (int)(r / M), m = (int)(r % M);
    ap[t] = A + w * a_ws + (long long)m * lda + kc;
  }
  const uint16_t *bp = wt + (long long)(n0 + (lane & 15)) * Kp + kc;
  v4f acc[2][4];
#pragma unroll
  for (int t = 0; t < 2; t++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[t][j] = (v4f){0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < Kp; k += 32) {
    const bool in = k + kc < Kp;  // Kp % 8 == 0: a lane's 8-half chunk is all in or all out
    v8h a[2], b[4];
#pragma unroll
    for (int t = 0; t < 2; t++) a[t] = in ? *(const v8h *)(ap[t] + k) : (v8h){};
#pragma unroll
    for (int j = 0; j < 4; j++) b[j] = in ? *(const v8h *)(bp + (long long)16 * j * Kp + k) : (v8h){};
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], b[j], acc[t][j], 0, 0, 0);
  }
  // accumulator lane layout: acc[t][j][r] = row 16 t + 4 (lane >> 4) + r, channel 16 j + (lane & 15)
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int n = n0 + 16 * j + (lane & 15);
    if (n >= Np || n >= e.ldo) continue;
    const float bn = bias[n];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const long long row = row0 + 16 * t + 4 * (lane >> 4) + r;
        if (row >= rows) continue;
        const int w = (int)(row / M), m = (int)(row % M);
        h16 v = f2h(acc[t][j][r] + bn);  // fp32 add, then one rounding to fp16 (nearest even)
        if (e.act == 1) v = silu_lut_h(v);
        else if (e.act == 2) v = hmax(v, (h16)0.0f);
        if (e.res) v = v + hfrom(e.res[w * e.res_ws + (long long)m * e.ldr + n]);
        long long orow = m;
        if (e.opad) orow = (long long)((m / e.ow) + e.opad) * (e.ow + 2 * e.opad) + (m % e.ow) + e.opad;
        e.out[w * e.out_ws + orow * e.ldo + n] = hbits(v);
      }
  }
}

// The same GEMM with the reference's own arithmetic (src/gemm_f16.c:49-171), so the outputs are bit-identical: per
// output an fp16 FMA chain over each K block (kblocks: ceil(Kp / 128) blocks, balanced, multiples of 8) from +0,
// the block results summed in fp32 when there are several (then + the fp32 bias, one rounding), else + the fp16
// bias in fp16; then the epilogue above. No MFMA (its accumulation is fp32): packed fp16 FMAs on the VALU, each
// lane one IEEE fp16 fused multiply-add, two channels per instruction.
// A block owns 64 rows x 128 channels; a thread 4 rows x 8 channels (16 packed accumulators). K is staged through
// LDS 32 at a time, A transposed to [k][row] and W as [k][channel], so a thread reads its 4 rows and 8 channels
// of a k step with one 8-byte and one 16-byte LDS read.
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#define FX_KC 32
__global__ __launch_bounds__(256) void k_gemm_f16x(const uint16_t *__restrict__ A, long long a_ws, int lda, int M,
                                                   double rM, long long rows, const uint16_t *__restrict__ wt,
                                                   const float *__restrict__ b32, const uint16_t *__restrict__ b16,
                                                   int Kp, int Np, int bs, Epi16Dev e) {
  __shared__ __attribute__((aligned(16))) h16 As[FX_KC][64 + 4];
  __shared__ __attribute__((aligned(16))) h16 Ws[FX_KC][128 + 8];
  __shared__ long long s_a[64], s_o[64], s_r[64];
  const int tid = threadIdx.x, tc = tid & 15, tr = tid >> 4;
  const long long rowB = (long long)blockIdx.x * 64;
  const int n0 = blockIdx.y * 128;
  if (tid < 64) {
    const long long row = rowB + tid < rows ? rowB + tid : rows - 1;
    const int w = bnh_div(row, M, rM), m = (int)(row - (long long)w * M);
    s_a[tid] = w * a_ws + (long long)m * lda;
    long long orow = m;
    if (e.opad) {
      const int y = m / e.ow;
      orow = (long long)(y + e.opad) * (e.ow + 2 * e.opad) + (m - y * e.ow) + e.opad;
    }
    s_o[tid] = w * e.out_ws + orow * e.ldo;
    s_r[tid] = w * e.res_ws + (long long)m * e.ldr;
  }
  __syncthreads();
  const int nblk = (Kp + bs - 1) / bs;
  h2 acc[4][4];
  float fb[4][8];
#pragma unroll
  for (int r = 0; r < 4; r++)
#pragma unroll
    for (int c = 0; c < 8; c++) fb[r][c] = 0.f;
  for (int kb = 0; kb < Kp; kb += bs) {
    const int ke = kb + bs < Kp ? kb + bs : Kp;
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int p = 0; p < 4; p++) acc[r][p] = (h2){(h16)0.0f, (h16)0.0f};
    for (int k0 = kb; k0 < ke; k0 += FX_KC) {
      const int kn = ke - k0 < FX_KC ? ke - k0 : FX_KC;  // a multiple of 8
      // stage A: 64 rows x kn k (8-half chunks), transposed
      for (int i = tid; i < 64 * (kn / 8); i += 256) {
        const int r = i / (kn / 8), kc = (i % (kn / 8)) * 8;
        const uint4 v = *(const uint4 *)(A + s_a[r] + k0 + kc);
        const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          As[kc + 2 * j][r] = hfrom((uint16_t)(q[j] & 0xffffu));
          As[kc + 2 * j + 1][r] = hfrom((uint16_t)(q[j] >> 16));
        }
      }
      // stage W: 128 channel rows x kn k
      for (int i = tid; i < 128 * (kn / 8); i += 256) {
        const int cch = i / (kn / 8), kc = (i % (kn / 8)) * 8;
        const uint4 v = *(const uint4 *)(wt + (long long)(n0 + cch) * Kp + k0 + kc);
        const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          Ws[kc + 2 * j][cch] = hfrom((uint16_t)(q[j] & 0xffffu));
          Ws[kc + 2 * j + 1][cch] = hfrom((uint16_t)(q[j] >> 16));
        }
      }
      __syncthreads();
      for (int k = 0; k < kn; k++) {
        const uint2 av = *(const uint2 *)&As[k][4 * tr];
        const uint4 wv = *(const uint4 *)&Ws[k][8 * tc];
        const h16 a[4] = {hfrom((uint16_t)(av.x & 0xffffu)), hfrom((uint16_t)(av.x >> 16)),
                          hfrom((uint16_t)(av.y & 0xffffu)), hfrom((uint16_t)(av.y >> 16))};
        const h2 w2[4] = {__builtin_bit_cast(h2, wv.x), __builtin_bit_cast(h2, wv.y), __builtin_bit_cast(h2, wv.z),
                          __builtin_bit_cast(h2, wv.w)};
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const h2 ar = (h2){a[r], a[r]};
#pragma unroll
          for (int p = 0; p < 4; p++) acc[r][p] = __builtin_elementwise_fma(w2[p], ar, acc[r][p]);
        }
      }
      __syncthreads();
    }
    if (nblk > 1) {
#pragma unroll
      for (int r = 0; r < 4; r++)
#pragma unroll
        for (int p = 0; p < 4; p++) {
          fb[r][2 * p] = fb[r][2 * p] + (float)acc[r][p].x;
          fb[r][2 * p + 1] = fb[r][2 * p + 1] + (float)acc[r][p].y;
        }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int lr = 4 * tr + r;
    if (rowB + lr >= rows) continue;
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const int n = n0 + 8 * tc + c;
      if (n >= Np || n >= e.ldo) continue;
      const h16 a = (c & 1) ? acc[r][c >> 1].y : acc[r][c >> 1].x;
      h16 v = nblk > 1 ? f2h(fb[r][c] + b32[n]) : a + hfrom(b16[n]);
      if (e.act == 1) v = silu_lut_h(v);
      else if (e.act == 2) v = hmax(v, (h16)0.0f);
      if (e.res) v = v + hfrom(e.res[s_r[lr] + n]);
      e.out[s_o[lr] + n] = hbits(v);
    }
  }
}

extern "C" {

bnh_h16w *bnh_h16w_new(int N, int K, int Kp, int Np, const uint16_t *w, const float *b32, const uint16_t *b16) {
  if (N <= 0 || K <= 0 || Np != ((N + 7) & ~7) || Kp < K || Kp % 8 || !w || !b32) {
    bnh_fail("bnh_h16w_new: fp16 GEMM shape N %d K %d Kp %d Np %d: expected Np = N rounded up to 8, Kp >= K, "
             "Kp %% 8 == 0, and both tensors", N, K, Kp, Np);
    return nullptr;
  }
  const int Nt = (int)bnh_round_up(Np, 128), n16 = Np / 16;
  uint16_t *hw = (uint16_t *)calloc((size_t)Nt * Kp, 2), *hb16 = (uint16_t *)calloc(Nt, 2);
  float *hb = (float *)calloc(Nt, 4);
  bnh_h16w *W = (bnh_h16w *)calloc(1, sizeof *W);
  if (!hw || !hb || !hb16 || !W) {
    free(hw); free(hb); free(hb16); free(W);
    bnh_fail("bnh_h16w_new: out of host memory");
    return nullptr;
  }
  for (int n = 0; n < Np; n++)  // hp_pack's layout (src/gemm_f16.c:18-40)
    for (int k = 0; k < Kp; k++) {
      const int nb = n / 16;
      const size_t idx = nb < n16 ? ((size_t)nb * Kp + k) * 16 + n % 16 : (size_t)n16 * Kp * 16 + (size_t)k * 8 + n % 16;
      hw[(size_t)n * Kp + k] = w[idx];
    }
  memcpy(hb, b32, sizeof(float) * Np);
  for (int n = 0; n < Np; n++) {  // the package's fp16 bias, or the fp32 one rounded to nearest even
    if (b16) hb16[n] = b16[n];
    else {
      const _Float16 h = (_Float16)b32[n];
      memcpy(&hb16[n], &h, 2);
    }
  }
  W->N = N; W->K = K; W->Kp = Kp; W->Np = Np; W->Nt = Nt;
  bool ok = (W->w = (uint16_t *)bnh_malloc((size_t)Nt * Kp * 2)) && (W->b = (float *)bnh_malloc(4 * (size_t)Nt)) &&
            (W->b16 = (uint16_t *)bnh_malloc(2 * (size_t)Nt)) &&
            !bnh_memcpy_h2d(W->w, hw, (size_t)Nt * Kp * 2) && !bnh_memcpy_h2d(W->b, hb, 4 * (size_t)Nt) &&
            !bnh_memcpy_h2d(W->b16, hb16, 2 * (size_t)Nt);
  free(hw); free(hb); free(hb16);
  if (!ok) { bnh_h16w_free(W); return nullptr; }
  return W;
}

void bnh_h16w_free(bnh_h16w *W) {
  if (!W) return;
  if (W->w) (void)hipFree(W->w);
  if (W->b) (void)hipFree(W->b);
  if (W->b16) (void)hipFree(W->b16);
  free(W);
}

static int gemm_f16_check(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W,
                          const bnh_epi16 *e) {
  BNH_REQ(A && W && e && e->out && M > 0 && B > 0 && lda >= W->Kp);
  BNH_REQ(((uintptr_t)A & 15) == 0 && lda % 8 == 0 && (B == 1 || a_ws % 8 == 0));
  BNH_REQ(e->act >= 0 && e->act <= 2 && e->ldo >= W->Np && e->opad >= 0 && e->opad <= 3);
  BNH_REQ(!e->opad || (e->ow > 0 && M % e->ow == 0));
  BNH_REQ(!e->res || e->ldr >= W->Np);
  BNH_REQ(!e->opad || B == 1 || e->out_ws >= (long long)(M / e->ow + 2 * e->opad) * (e->ow + 2 * e->opad) * e->ldo);
  return 0;
}

static int zero_halo16(const bnh_epi16 *e, int M, int B, void *stream) {
  if (!e->opad) return 0;
  const int H = M / e->ow;
  const long long per = (long long)(H + 2 * e->opad) * (e->ow + 2 * e->opad) * e->ldo;
  return bnh_zero_halo(e->out, B == 1 ? per : e->out_ws, H, e->ow, e->ldo, e->opad, 2, B, stream);
}

int bnh_gemm_f16_body(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W, const bnh_epi16 *e,
                      void *stream) {
  if (gemm_f16_check(A, a_ws, lda, M, B, W, e)) return -1;
  const long long rows = (long long)M * B;
  Epi16Dev d = {e->act, e->out, e->out_ws, e->ldo, e->ow, e->opad, e->res, e->res_ws, e->ldr};
  const int nblk = (W->Kp + 127) / 128, bs = ((W->Kp + nblk - 1) / nblk + 7) & ~7;  // kblocks (src/gemm_f16.c:55-58)
  dim3 grid((unsigned)bnh_ceil_div(rows, 64), (unsigned)bnh_ceil_div(W->Np, 128));
  hipLaunchKernelGGL(k_gemm_f16x, grid, dim3(256), 0, bnh_stream(stream), A, a_ws, lda, M, 1.0 / M, rows, W->w, W->b,
                     W->b16, W->Kp, W->Np, bs, d);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_gemm_f16(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W, const bnh_epi16 *e,
                 void *stream) {
  if (gemm_f16_check(A, a_ws, lda, M, B, W, e) || zero_halo16(e, M, B, stream)) return -1;
  return bnh_gemm_f16_body(A, a_ws, lda, M, B, W, e, stream);
}

int bnh_gemm_f16_mfma(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W, const bnh_epi16 *e,
                      void *stream) {
  if (gemm_f16_check(A, a_ws, lda, M, B, W, e) || zero_halo16(e, M, B, stream)) return -1;
  const long long rows = (long long)M * B;
  Epi16Dev d = {e->act, e->out, e->out_ws, e->ldo, e->ow, e->opad, e->res, e->res_ws, e->ldr};
  dim3 grid((unsigned)bnh_ceil_div(rows, 64), (unsigned)bnh_ceil_div(W->Np, 128));
  hipLaunchKernelGGL(k_gemm_f16, grid, dim3(256), 0, bnh_stream(stream), A, a_ws, lda, M, rows, W->w, W->b, W->Kp,
                     W->Np, d);
  BNH_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
