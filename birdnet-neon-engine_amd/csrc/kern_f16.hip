// fp16 pointwise-convolution GEMM (libbnneon's gemm_f16, src/gemm_f16.c, the PW op of the fp16 family) on gfx950
// fp16 MFMA (v_mfma_f32_16x16x32_f16): fp16 operands, fp32 accumulation over the whole K, then the reference's
// epilogue in its own arithmetic: + bias in fp32, one rounding to fp16, fp16 LUT SiLU or ReLU, fp16 residual add,
// zero-haloed store. The reference accumulates in fp16 within K blocks of <= 128 steps; the fp32 accumulation here
// is the more accurate of the two and stays within the fp16 accumulation error bound of the reference's result (the
// tolerance the parity tests state).
//
// Layouts: A fp16 NHWC rows [M][lda] per window (k contiguous: lane l of an MFMA takes 8 halves of row (l & 15) at
// k offset 8 (l >> 4)); weights repacked at load from the package's [Np/16][Kp][16] + [Kp][8] panels into channel
// rows [Nt][Kp] (Nt = Np rounded to 128, zero rows past Np); fp32 bias [Nt].
#include <string.h>

#include "bnh_internal.h"
#include "bnh_num.h"
#include "bnh_f16.h"

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

struct bnh_h16w {
  int N, K, Kp, Np, Nt;
  uint16_t *w;  // [Nt][Kp]
  float *b;     // [Nt]
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

// zero halo of a padded fp16 output (rt_zero_halo with 2-byte elements), every window
__global__ void k_zero_halo_u16(uint16_t *__restrict__ out, long long ws, int H, int W, int C, int h, long long total) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int Wp = W + 2 * h;
  const long long per = (long long)(H + 2 * h) * Wp * C;
  const int w = (int)(i / per);
  const long long el = i % per, px = el / C;
  const int y = (int)(px / Wp), x = (int)(px % Wp);
  if (y >= h && y < H + h && x >= h && x < W + h) return;
  out[w * ws + el] = 0;
}

extern "C" {

bnh_h16w *bnh_h16w_new(int N, int K, int Kp, int Np, const uint16_t *w, const float *b32) {
  if (N <= 0 || K <= 0 || Np != ((N + 7) & ~7) || Kp < K || Kp % 8 || !w || !b32) {
    bnh_fail("bnh_h16w_new: fp16 GEMM shape N %d K %d Kp %d Np %d: expected Np = N rounded up to 8, Kp >= K, "
             "Kp %% 8 == 0, and both tensors", N, K, Kp, Np);
    return nullptr;
  }
  const int Nt = (int)bnh_round_up(Np, 128), n16 = Np / 16;
  uint16_t *hw = (uint16_t *)calloc((size_t)Nt * Kp, 2);
  float *hb = (float *)calloc(Nt, 4);
  bnh_h16w *W = (bnh_h16w *)calloc(1, sizeof *W);
  if (!hw || !hb || !W) {
    free(hw); free(hb); free(W);
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
  W->N = N; W->K = K; W->Kp = Kp; W->Np = Np; W->Nt = Nt;
  bool ok = (W->w = (uint16_t *)bnh_malloc((size_t)Nt * Kp * 2)) && (W->b = (float *)bnh_malloc(4 * (size_t)Nt)) &&
            !bnh_memcpy_h2d(W->w, hw, (size_t)Nt * Kp * 2) && !bnh_memcpy_h2d(W->b, hb, 4 * (size_t)Nt);
  free(hw); free(hb);
  if (!ok) { bnh_h16w_free(W); return nullptr; }
  return W;
}

void bnh_h16w_free(bnh_h16w *W) {
  if (!W) return;
  if (W->w) (void)hipFree(W->w);
  if (W->b) (void)hipFree(W->b);
  free(W);
}

int bnh_gemm_f16(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W, const bnh_epi16 *e,
                 void *stream) {
  BNH_REQ(A && W && e && e->out && M > 0 && B > 0 && lda >= W->Kp);
  BNH_REQ(((uintptr_t)A & 15) == 0 && lda % 8 == 0 && (B == 1 || a_ws % 8 == 0));
  BNH_REQ(e->act >= 0 && e->act <= 2 && e->ldo >= W->Np && e->opad >= 0 && e->opad <= 3);
  BNH_REQ(!e->opad || (e->ow > 0 && M % e->ow == 0));
  BNH_REQ(!e->res || e->ldr >= W->Np);
  hipStream_t st = bnh_stream(stream);
  if (e->opad) {
    const int H = M / e->ow, h = e->opad;
    const long long per = (long long)(H + 2 * h) * (e->ow + 2 * h) * e->ldo, total = per * B;
    BNH_REQ(B == 1 || e->out_ws >= per);
    hipLaunchKernelGGL(k_zero_halo_u16, dim3((unsigned)bnh_ceil_div(total, 256)), dim3(256), 0, st, e->out,
                       B == 1 ? per : e->out_ws, H, e->ow, e->ldo, h, total);
    BNH_HIP(hipGetLastError());
  }
  const long long rows = (long long)M * B;
  Epi16Dev d = {e->act, e->out, e->out_ws, e->ldo, e->ow, e->opad, e->res, e->res_ws, e->ldr};
  dim3 grid((unsigned)bnh_ceil_div(rows, 64), (unsigned)bnh_ceil_div(W->Np, 128));
  hipLaunchKernelGGL(k_gemm_f16, grid, dim3(256), 0, st, A, a_ws, lda, M, rows, W->w, W->b, W->Kp, W->Np, d);
  BNH_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
