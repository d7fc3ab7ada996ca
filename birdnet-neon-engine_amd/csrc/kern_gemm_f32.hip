// fp32 1x1 convolution / GEMM of the registry's PW op (src/rt_ops_f32.c:129-212, gemm_f32 / gemm_f32_range_gate
// src/gemm_f32.c:141-197), bit-identical: every output (m, n), n < Np, is one fp32 FMA chain over k < Kp from +0 in
// k order (the 8 x 8 register tile's chains, src/gemm_f32_kblock.h), + b[n], the activation (the NEON SiLU / max 0),
// + residual, stored at its padded row; a gated A is the fp32 product A[m][k] gate[k] (the value an in-place gating
// multiply stores). No MFMA: the matrix cores sum their products in an order of their own.
//
// Tiling: a block of 256 threads owns 64 rows x 64 channels of one window; K goes in chunks of 16 through LDS (A
// transposed to [k][m], the package panels' [k][8] rows side by side as [k][n]); thread (ty, tx) owns rows ty + 16 i
// and channels 4 tx + j (i, j < 4), so each k step is 4 LDS reads of A (shared by the 16 lanes of a row group),
// one 16-byte read of W and 16 FMAs.
#include "bnh_internal.h"
#include "bnh_num.h"

#define GF_TM 64
#define GF_TN 64
#define GF_KC 16

__global__ __launch_bounds__(256) void k_gemm_f32(const float *__restrict__ A, long long a_ws, int lda, int M, int Kp,
                                                  const float *__restrict__ gate, long long g_ws,
                                                  const float *__restrict__ w, const float *__restrict__ bias, int Np,
                                                  bnh_epi32 e) {
  __shared__ float As[GF_KC][GF_TM + 4];
  __shared__ __attribute__((aligned(16))) float Ws[GF_KC][GF_TN + 4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int win = blockIdx.z, m0 = blockIdx.x * GF_TM, n0 = blockIdx.y * GF_TN;
  const float *Aw = A + win * a_ws;
  const float *gw = gate ? gate + win * g_ws : nullptr;
  // this thread's loads per chunk: A row ar, k ak..ak+3; W panel wp, k row wk, entries we..we+3
  const int ar = tid >> 2, ak = (tid & 3) * 4;
  const int wp = tid >> 5, wk = (tid & 31) >> 1, we = (tid & 1) * 4;
  const bool a_ok = m0 + ar < M, w_ok = n0 + 8 * wp < Np;
  const float *arow = Aw + (long long)(m0 + ar) * lda;
  const float *wpan = w + (long long)(n0 / 8 + wp) * Kp * 8;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = 0.f;
  for (int k0 = 0; k0 < Kp; k0 += GF_KC) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int k = k0 + ak + q;
      float a = 0.f;
      if (a_ok && k < Kp) {
        a = arow[k];
        if (gw) a = a * gw[k];
      }
      As[ak + q][ar] = a;
    }
    float4 wv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (w_ok && k0 + wk < Kp) wv = *(const float4 *)(wpan + (long long)(k0 + wk) * 8 + we);
    *(float4 *)&Ws[wk][8 * wp + we] = wv;
    __syncthreads();
    const int kn = Kp - k0 < GF_KC ? Kp - k0 : GF_KC;
    if (kn == GF_KC) {
#pragma unroll
      for (int kk = 0; kk < GF_KC; kk++) {
        const float4 b4 = *(const float4 *)&Ws[kk][4 * tx];
        const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float a = As[kk][ty + 16 * i];
#pragma unroll
          for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(a, bv[j], acc[i][j]);
        }
      }
    } else {  // the last chunk of a Kp that is not a multiple of 16: the chains stop at Kp
      for (int kk = 0; kk < kn; kk++) {
        const float4 b4 = *(const float4 *)&Ws[kk][4 * tx];
        const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float a = As[kk][ty + 16 * i];
#pragma unroll
          for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(a, bv[j], acc[i][j]);
        }
      }
    }
    __syncthreads();
  }
  // epilogue: + b, activation, + residual, padded store
  float *ow = e.out + win * e.out_ws;
  const float *rw = e.res ? e.res + win * e.res_ws : nullptr;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int m = m0 + ty + 16 * i;
    if (m >= M) continue;
    const long long orow = e.opad ? (long long)(m / e.ow + e.opad) * (e.ow + 2 * e.opad) + m % e.ow + e.opad : m;
    const long long rrow = e.rpad ? (long long)(m / e.rw + e.rpad) * (e.rw + 2 * e.rpad) + m % e.rw + e.rpad : m;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + 4 * tx + j;
      if (n >= Np) continue;
      float y = acc[i][j] + bias[n];
      if (e.act == 1) y = bnh_silu_f32(y);
      else if (e.act == 2) y = bnh_relu_f32(y);
      if (rw) y = y + rw[rrow * e.ldr + n];
      ow[orow * e.ldo + n] = y;
    }
  }
}

extern "C" int bnh_gemm_f32(const float *A, long long a_ws, int lda, int M, const float *gate, long long g_ws,
                            const float *w, const float *bias, int Kp, int Np, const bnh_epi32 *e, int B,
                            void *stream) {
  BNH_REQ(A && w && bias && e && e->out && M > 0 && B > 0 && B <= 65535);
  BNH_REQ(Kp > 0 && Kp % 4 == 0 && Np > 0 && Np % 8 == 0 && lda >= Kp && e->ldo >= Np);
  BNH_REQ(e->act >= 0 && e->act <= 2 && e->opad >= 0 && e->opad <= 3 && (!e->opad || (e->ow > 0 && M % e->ow == 0)));
  BNH_REQ(!e->res || (e->ldr >= Np && (!e->rpad || (e->rw > 0 && M % e->rw == 0))));
  BNH_REQ(((uintptr_t)w & 15) == 0);
  BNH_REQ(B == 1 || (a_ws >= (long long)M * lda && (!gate || g_ws >= Kp)));
  const dim3 grid((unsigned)bnh_ceil_div(M, GF_TM), (unsigned)bnh_ceil_div(Np, GF_TN), (unsigned)B);
  hipLaunchKernelGGL(k_gemm_f32, grid, dim3(256), 0, bnh_stream(stream), A, a_ws, lda, M, Kp, gate, g_ws, w, bias, Np,
                     *e);
  BNH_HIP(hipGetLastError());
  return 0;
}
