// fp32 registry ops around the int8 GEMMs of the int8 Perch-family plan, bit-identical to libbnneon's fp32 kernels:
//   STEM     im2col of a 1-channel image (VALID k x k, stride s) into the fp32 GEMM (src/rt_ops_f32.c:409-425,
//            pc_im2col1 src/pc_kern_f32.c:150-161, gemm_f32 src/gemm_f32.c:141-197): per output one FMA chain over
//            the Kp taps from +0, + bias, SiLU / ReLU, padded store;
//   SE_GATE  the squeeze-excitation gate from the depthwise conv's channel sums (src/rt_ops_f32.c:317-324 with
//   / SE     v24k32_se_fc1 src/v24_f32.c:164-179 and se_gate_range src/rt_ops_f32.c:269-283), SE also gating the
//            activation in place (v24k32_se, src/v24_f32.c:181-210);
//   MEAN     spatial mean (pc_mean_f32, src/pc_kern_f32.c:342-348);
//   PAD      copy into a zero-haloed buffer (src/rt_ops_f32.c:503-508), fp32 or fp16;
// and the halo zeroing every padded output needs (rt_zero_halo, src/rt_pkg.c:194-203).
#include <string.h>

#include "bnh_internal.h"
#include "bnh_num.h"
#include "bnh_expf.h"
#include "bnh_powf.h"
#include "bnh_f16.h"

// ------------------------------------------------------------------ halo zeroing, any element size (4 or 2 bytes)
// one thread per halo element: the 2h rows of Wp pixels above and below, then the 2h side pixels of each interior row
template <typename T>
__global__ void k_zero_halo(T *__restrict__ out, long long ws, int H, int W, int C, int h, long long total) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int Wp = W + 2 * h;
  const long long nh = 2LL * h * (Wp + H) * C;
  const int win = (int)(i / nh);
  const long long e = i % nh;
  const int c = (int)(e % C);
  const long long hp = e / C;
  int y, x;
  if (hp < 2LL * h * Wp) {
    const int t = (int)(hp / Wp);
    x = (int)(hp % Wp);
    y = t < h ? t : H + t;
  } else {
    const int u = (int)(hp - 2LL * h * Wp), sd = u % (2 * h);
    y = h + u / (2 * h);
    x = sd < h ? sd : W + sd;
  }
  out[win * ws + ((long long)y * Wp + x) * C + c] = (T)0;
}

// ------------------------------------------------------------------ STEM
// thread per (window, output pixel, 4 channels); w panels [Np/8][Kp][8]. H16: the fp16-path form, channels < N
// rounded to fp16 (pc_cvt_pad_f16, src/pc_kern_f16.c:104-113) and stored as fp16
// KK: the kernel size when it is 3 or 5 (the taps unrolled), 0 for any k. A thread owns 4 output channels of one
// pixel; windows on grid.y; 32-bit index arithmetic; 16-byte stores when the output rows allow them (VEC). The
// weight panels and the bias are copied into LDS once per block (dynamic LDS, Np Kp + Np floats): every thread reads
// Kp 16-byte weight rows, the same for every pixel, which through the vector memory path bound the kernel on its
// address units.
// NPX > 1 (3 x 3 taps): a thread owns 4 output channels of NPX pixels m, m + MQ, ... (MQ = ceil(Ho Wo / NPX)),
// with the channels' 12 weight rows read from LDS into registers once (not once per pixel) and the block's set-up
// (the SiLU table, the panels in LDS) spread over NPX times the pixels.
template <int KK, bool H16, bool VEC, int NPX>
__global__ __launch_bounds__(256) void k_stem_f32(const float *__restrict__ img, long long i_ws, int W, int k, int s,
                                                  int Ho, int Wo, const float *__restrict__ w,
                                                  const float *__restrict__ bias, int Kp, int Np, int act,
                                                  void *__restrict__ outv, long long o_ws, int ldo, int opad, int N) {
  __shared__ uint32_t tbl[256];
  extern __shared__ __attribute__((aligned(16))) float s_wb[];  // [Np Kp] panels, then [Np] bias
  bnh_silu_table(tbl);
  for (int i = threadIdx.x; i < Np * Kp / 4; i += blockDim.x) ((float4 *)s_wb)[i] = ((const float4 *)w)[i];
  for (int i = threadIdx.x; i < Np; i += blockDim.x) s_wb[Np * Kp + i] = bias[i];
  __syncthreads();
  const int ng = Np / 4, npx = Ho * Wo, MQ = (npx + NPX - 1) / NPX;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const long long win = blockIdx.y;
  if (i >= MQ * ng) return;
  const int mq = i / ng, g = i - mq * ng, n0 = 4 * g;
  const float *wp = s_wb + (n0 / 8) * Kp * 8 + n0 % 8;
  constexpr int KP = KK > 0 ? (KK * KK + 3) / 4 * 4 : 1;
  float4 wr[NPX > 1 ? KP : 1];
  if constexpr (NPX > 1) {
#pragma unroll
    for (int q = 0; q < KP; q++) wr[q] = *(const float4 *)(wp + q * 8);
  }
#pragma unroll
  for (int j = 0; j < NPX; j++) {
    const int m = mq + j * MQ;
    if (m >= npx) break;
    const int oy = m / Wo, ox = m - oy * Wo;
    const float *x = img + win * i_ws + (oy * s) * W + ox * s;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    auto tap = [&](int q, float a) {
      const float4 wv = NPX > 1 ? wr[NPX > 1 ? q : 0] : *(const float4 *)(wp + q * 8);
      acc[0] = __builtin_fmaf(wv.x, a, acc[0]);
      acc[1] = __builtin_fmaf(wv.y, a, acc[1]);
      acc[2] = __builtin_fmaf(wv.z, a, acc[2]);
      acc[3] = __builtin_fmaf(wv.w, a, acc[3]);
    };
    if constexpr (KK > 0) {
      float a[KP];
#pragma unroll
      for (int q = 0; q < KP; q++) a[q] = q < KK * KK ? x[(q / KK) * W + q % KK] : 0.f;
#pragma unroll
      for (int q = 0; q < KP; q++) tap(q, a[q]);
    } else {
      for (int q = 0; q < Kp; q++) tap(q, q < k * k ? x[(q / k) * W + q % k] : 0.f);
    }
    float y[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      y[u] = acc[u] + s_wb[Np * Kp + n0 + u];
      if (act == 1) y[u] = bnh_silu_f32_t(y[u], tbl);
      else if (act == 2) y[u] = bnh_relu_f32(y[u]);
    }
    const long long orow = opad ? (long long)(oy + opad) * (Wo + 2 * opad) + ox + opad : m;
    if (H16) {
      uint16_t *o = (uint16_t *)outv + win * o_ws + orow * ldo + n0;
      if (VEC && n0 + 4 <= N) {
        *(uint2 *)o = make_uint2((uint32_t)hbits(f2h(y[0])) | ((uint32_t)hbits(f2h(y[1])) << 16),
                                 (uint32_t)hbits(f2h(y[2])) | ((uint32_t)hbits(f2h(y[3])) << 16));
      } else {
#pragma unroll
        for (int u = 0; u < 4; u++)
          if (n0 + u < N) o[u] = hbits(f2h(y[u]));  // one rounding to nearest even (no fused mix forms)
      }
    } else {
      float *o = (float *)outv + win * o_ws + orow * ldo + n0;
      if (VEC) {
        *(float4 *)o = make_float4(y[0], y[1], y[2], y[3]);
      } else {
        o[0] = y[0]; o[1] = y[1]; o[2] = y[2]; o[3] = y[3];
      }
    }
  }
}

// the stem launch for kernel size k: the unrolled forms for 3 and 5
template <bool H16>
static void stem_launch(dim3 grid, hipStream_t st, bool vec, const float *img, long long i_ws, int W, int k, int s,
                        int Ho, int Wo, const float *w, const float *bias, int Kp, int Np, int act, void *out,
                        long long o_ws, int ldo, int opad, int N) {
  const size_t lds = sizeof(float) * ((size_t)Np * Kp + Np);
  const long long ng = Np / 4, npx = (long long)Ho * Wo;
  auto g = [&](int npxt) { return dim3((unsigned)bnh_ceil_div(bnh_ceil_div(npx, npxt) * ng, 256), grid.y); };
#define STEM_L(KK, V, P)                                                                                               \
  hipLaunchKernelGGL((k_stem_f32<KK, H16, V, P>), g(P), dim3(256), lds, st, img, i_ws, W, k, s, Ho, Wo, w, bias, Kp,  \
                     Np, act, out, o_ws, ldo, opad, N)
  if (k == 3 && Kp == 12) { if (vec) STEM_L(3, true, 4); else STEM_L(3, false, 4); }
  else if (k == 5 && Kp == 28) { if (vec) STEM_L(5, true, 1); else STEM_L(5, false, 1); }
  else { if (vec) STEM_L(0, true, 1); else STEM_L(0, false, 1); }
#undef STEM_L
}

// ------------------------------------------------------------------ SE_GATE / SE
// The gate's sigmoid: sigmoid_f32x4 (src/gemm_f32.h:93-96), 1 / (1 + exp2_f32x4(-a log2 e)) by FRECPE and two
// Newton steps; F16: the fp16 path's sigm4 (src/v24_fast.c:182-195), the same 2^t divided into 1 (IEEE division)
template <bool F16>
BNH_DEV float se_sigmoid(float a) {
  float t = a * -1.44269504f;
  t = bnh_fmin(bnh_fmax(t, -126.f), 126.f);
  const float n = __builtin_rintf(t), f = t - n;
  float q = 1.5403530e-4f;
  q = __builtin_fmaf(q, f, 1.3333558e-3f);
  q = __builtin_fmaf(q, f, 9.6181291e-3f);
  q = __builtin_fmaf(q, f, 5.5504109e-2f);
  q = __builtin_fmaf(q, f, 2.4022651e-1f);
  q = __builtin_fmaf(q, f, 6.9314718e-1f);
  q = __builtin_fmaf(q, f, 1.f);
  const float e = bnh_float(bnh_bits(q) + ((uint32_t)bnh_cvtz_s32(n) << 23));
  const float d = 1.f + e;
  if (F16) return 1.f / d;
  float rr = bnh_frecpe(d);
  rr = rr * bnh_frecps(d, rr);
  return rr * bnh_frecps(d, rr);
}

// With a workspace the gates come from two kernels over all windows. k_se_fc1: a block per WB windows x 32 rows r of
// w1; thread (r, l) runs lane chain l (c = l, l + 8, ...; the K % 8 remainder in lanes 0-3, as two 4-lane
// accumulators over 8-channel steps do) for its WB windows; the chains are summed pairwise, + b1, SiLU by the C
// library's expf, into s1 [B][rd].
template <int WB>
__global__ __launch_bounds__(256) void k_se_fc1(const float *__restrict__ chsum, long long c_ws, int C, int rd, float inv,
                                                const float *__restrict__ w1, const float *__restrict__ b1,
                                                float *__restrict__ s1, int B) {
  extern __shared__ float sm[];
  float *mean = sm, *part = sm + WB * C;  // [WB][C], [WB][32][8]
  const int win0 = blockIdx.x * WB, nw = B - win0 < WB ? B - win0 : WB, r0 = blockIdx.y * 32, tid = threadIdx.x;
  for (int i = tid; i < WB * C; i += 256) {
    const int wg = i / C, c = i - wg * C;
    mean[i] = wg < nw ? chsum[(win0 + wg) * c_ws + c] * inv : 0.f;
  }
  __syncthreads();
  const int rl = tid / 8, l = tid % 8, r = r0 + rl, C8 = C / 8 * 8;
  if (r < rd) {
    const float *w = w1 + (long long)r * C;
    float a[WB];
#pragma unroll
    for (int wg = 0; wg < WB; wg++) a[wg] = 0.f;
    // 32 of the chain's weights loaded at once, then their FMAs in order (one memory round trip per 32 steps of the
    // chain, not per step; the launch has few waves, so the registers cost no occupancy that matters)
    for (int cb = l; cb < C8; cb += 8 * 32) {
      float wv[32];
#pragma unroll
      for (int u = 0; u < 32; u++) wv[u] = cb + 8 * u < C8 ? w[cb + 8 * u] : 0.f;
      float mv[32][WB];  // the means they multiply, read from LDS ahead of the chain too
#pragma unroll
      for (int u = 0; u < 32; u++)
#pragma unroll
        for (int wg = 0; wg < WB; wg++) mv[u][wg] = cb + 8 * u < C8 ? mean[wg * C + cb + 8 * u] : 0.f;
#pragma unroll
      for (int u = 0; u < 32; u++) {
        if (cb + 8 * u < C8) {
#pragma unroll
          for (int wg = 0; wg < WB; wg++) a[wg] = __builtin_fmaf(wv[u], mv[u][wg], a[wg]);
        }
      }
    }
    if (l < 4 && C8 + l < C) {
      const float wv = w[C8 + l];
#pragma unroll
      for (int wg = 0; wg < WB; wg++) a[wg] = __builtin_fmaf(wv, mean[wg * C + C8 + l], a[wg]);
    }
#pragma unroll
    for (int wg = 0; wg < WB; wg++) part[(wg * 32 + rl) * 8 + l] = a[wg];
  }
  __syncthreads();
  for (int i = tid; i < WB * 32; i += 256) {
    const int wg = i / 32, rr = r0 + i % 32;
    if (wg >= nw || rr >= rd) continue;
    const float *pp = part + i * 8;
    const float v = ((pp[0] + pp[4]) + (pp[1] + pp[5])) + ((pp[2] + pp[6]) + (pp[3] + pp[7]));
    const float x = v + b1[rr];
    s1[(long long)(win0 + wg) * rd + rr] = x / (1.f + bnh_expf(-x));  // silu_s: the C library's expf
  }
}

// k_se_fc2: a thread per channel c of WB windows: from b2, one FMA per row r, then the sigmoid, into gate
template <int WB, bool F16>
__global__ __launch_bounds__(256) void k_se_fc2(const float *__restrict__ s1, int C, int rd,
                                                const float *__restrict__ w2t, const float *__restrict__ b2,
                                                float *__restrict__ gate, long long g_ws, int B,
                                                uint16_t *__restrict__ gh, long long gh_ws) {
  extern __shared__ float ss[];  // [WB][rd]
  const int win0 = blockIdx.y * WB, nw = B - win0 < WB ? B - win0 : WB, tid = threadIdx.x;
  for (int i = tid; i < WB * rd; i += 256) ss[i] = i / rd < nw ? s1[(long long)win0 * rd + i] : 0.f;
  __syncthreads();
  const int c = blockIdx.x * 256 + tid;
  if (c >= C) return;
  float a[WB];
  const float b = b2[c];
#pragma unroll
  for (int wg = 0; wg < WB; wg++) a[wg] = b;
  for (int rb = 0; rb < rd; rb += 32) {  // 32 rows' weights loaded at once, then their FMAs in order
    float wv[32];
#pragma unroll
    for (int u = 0; u < 32; u++) wv[u] = rb + u < rd ? w2t[(long long)(rb + u) * C + c] : 0.f;
#pragma unroll
    for (int u = 0; u < 32; u++)
      if (rb + u < rd) {
#pragma unroll
        for (int wg = 0; wg < WB; wg++) a[wg] = __builtin_fmaf(wv[u], ss[wg * rd + rb + u], a[wg]);
      }
  }
#pragma unroll
  for (int wg = 0; wg < WB; wg++)
    if (wg < nw) {
      const float gv = se_sigmoid<F16>(a[wg]);
      gate[(win0 + wg) * g_ws + c] = gv;
      if (gh) gh[(win0 + wg) * gh_ws + c] = hbits(f2h(gv));  // the fp16 gate the scaling multiplies by
    }
}

// Without a workspace: one block per group of windows
// A block computes the gates of WG windows (so each weight it streams serves WG windows), every value with the
// reference's instructions in its order: mean = chsum * (1 / P); fc1 as eight lane chains (two 4-lane accumulators
// over 8-channel steps) summed pairwise, + b1, SiLU by the C library's expf; fc2 from b2, one FMA per row r;
// sigmoid_f32x4. SE also gates the activation [P][C] in place.
// F16: the fp16 path's SE (v24k16_se, src/v24_fast.c:182-234): its sigmoid divides (1 / (1 + e), IEEE division),
// the gate is rounded to fp16 and the fp16 activation is multiplied by it in fp16
template <int WG, bool F16>
__global__ __launch_bounds__(256) void k_se_f32(const float *__restrict__ chsum, long long c_ws, int C, int rd, int P,
                                                const float *__restrict__ w1, const float *__restrict__ b1,
                                                const float *__restrict__ w2t, const float *__restrict__ b2,
                                                float *__restrict__ gate, long long g_ws, void *__restrict__ Dv,
                                                long long d_ws, int B) {
  extern __shared__ float sm[];
  float *mean = sm, *part = sm + WG * C, *s1 = part + WG * 8 * rd, *g = s1 + WG * rd;  // [WG][C] [WG][rd][8] [WG][rd]
  const int win0 = blockIdx.x * WG, nw = B - win0 < WG ? B - win0 : WG, tid = threadIdx.x;
  const float inv = 1.f / (float)P;
  for (int i = tid; i < WG * C; i += 256) {
    const int wg = i / C, c = i - wg * C;
    mean[i] = wg < nw ? chsum[(win0 + wg) * c_ws + c] * inv : 0.f;
  }
  __syncthreads();
  const int C8 = C / 8 * 8;
  for (int it = tid; it < 8 * rd; it += 256) {
    const int r = it / 8, l = it % 8;
    const float *w = w1 + (long long)r * C;
    float a[WG];
#pragma unroll
    for (int wg = 0; wg < WG; wg++) a[wg] = 0.f;
#pragma unroll 8
    for (int c = l; c < C8; c += 8) {
      const float wv = w[c];
#pragma unroll
      for (int wg = 0; wg < WG; wg++) a[wg] = __builtin_fmaf(wv, mean[wg * C + c], a[wg]);
    }
    if (l < 4 && C8 + l < C) {
      const float wv = w[C8 + l];
#pragma unroll
      for (int wg = 0; wg < WG; wg++) a[wg] = __builtin_fmaf(wv, mean[wg * C + C8 + l], a[wg]);
    }
#pragma unroll
    for (int wg = 0; wg < WG; wg++) part[(wg * rd + r) * 8 + l] = a[wg];
  }
  __syncthreads();
  for (int i = tid; i < WG * rd; i += 256) {
    const int r = i % rd;
    const float *pp = part + i * 8;
    const float v = ((pp[0] + pp[4]) + (pp[1] + pp[5])) + ((pp[2] + pp[6]) + (pp[3] + pp[7]));
    const float x = v + b1[r];
    s1[i] = x / (1.f + bnh_expf(-x));  // silu_s: the C library's expf
  }
  __syncthreads();
  for (int c = tid; c < C; c += 256) {
    float a[WG];
    const float b = b2[c];
#pragma unroll
    for (int wg = 0; wg < WG; wg++) a[wg] = b;
#pragma unroll 8
    for (int r = 0; r < rd; r++) {
      const float wv = w2t[(long long)r * C + c];
#pragma unroll
      for (int wg = 0; wg < WG; wg++) a[wg] = __builtin_fmaf(wv, s1[wg * rd + r], a[wg]);
    }
#pragma unroll
    for (int wg = 0; wg < WG; wg++) {
      const float rr = se_sigmoid<F16>(a[wg]);
      g[wg * C + c] = rr;
      if (gate && wg < nw) gate[(win0 + wg) * g_ws + c] = rr;
    }
  }
  if (!Dv) return;
  __syncthreads();
  for (int wg = 0; wg < nw; wg++) {
    const float *gg = g + wg * C;
    if (F16) {
      h16 *d = (h16 *)Dv + (win0 + wg) * d_ws;
      for (long long i = tid; i < (long long)P * C; i += 256) d[i] = d[i] * f2h(gg[i % C]);
    } else {
      float *d = (float *)Dv + (win0 + wg) * d_ws;
      for (long long i = tid; i < (long long)P * C; i += 256) d[i] = d[i] * gg[i % C];
    }
  }
}

// SE scaling when the gates are in a buffer: D[p][c] *= gate[c] for every window, 8 channels per thread (C % 8 == 0)
// over a grid that covers all windows; fp16: the gate rounded to fp16, the product in fp16 (v24k16_se_scale,
// src/v24_fast.c:223-228); fp32: the fp32 product. VEC: 16-byte vector accesses (aligned strides), else scalar.
template <bool F16, bool VEC>
__global__ __launch_bounds__(256) void k_se_scale(const float *__restrict__ gate, long long g_ws, int C, long long n8,
                                                  void *__restrict__ Dv, long long d_ws) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const long long win = blockIdx.y, e = i * 8;
  const int c = (int)(e % C);
  const float *g = gate + win * g_ws + c;
  float gv[8];
  if (VEC) {
    const float4 g0 = *(const float4 *)g, g1 = *(const float4 *)(g + 4);
    gv[0] = g0.x; gv[1] = g0.y; gv[2] = g0.z; gv[3] = g0.w; gv[4] = g1.x; gv[5] = g1.y; gv[6] = g1.z; gv[7] = g1.w;
  } else {
#pragma unroll
    for (int j = 0; j < 8; j++) gv[j] = g[j];
  }
  if (F16) {
    uint16_t *d = (uint16_t *)Dv + win * d_ws + e;
    if (VEC) {
      uint4 v = *(const uint4 *)d;
      uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const h16 lo = hfrom((uint16_t)(q[j] & 0xffffu)) * f2h(gv[2 * j]);
        const h16 hi = hfrom((uint16_t)(q[j] >> 16)) * f2h(gv[2 * j + 1]);
        q[j] = (uint32_t)hbits(lo) | ((uint32_t)hbits(hi) << 16);
      }
      *(uint4 *)d = make_uint4(q[0], q[1], q[2], q[3]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) d[j] = hbits(hfrom(d[j]) * f2h(gv[j]));
    }
  } else {
    float *d = (float *)Dv + win * d_ws + e;
    if (VEC) {
      float4 a = *(const float4 *)d, b = *(const float4 *)(d + 4);
      a.x *= gv[0]; a.y *= gv[1]; a.z *= gv[2]; a.w *= gv[3];
      b.x *= gv[4]; b.y *= gv[5]; b.z *= gv[6]; b.w *= gv[7];
      *(float4 *)d = a;
      *(float4 *)(d + 4) = b;
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) d[j] = d[j] * gv[j];
    }
  }
}

// ------------------------------------------------------------------ MEAN
__global__ void k_mean_f32(const float *__restrict__ x, long long x_ws, int P, int C, int ld, float *__restrict__ out,
                           long long o_ws) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x, win = blockIdx.y;
  if (c >= C) return;
  const float *xw = x + win * x_ws + c;
  float s = 0.f;
  for (int p = 0; p < P; p++) s = s + xw[(long long)p * ld];
  out[win * o_ws + c] = s / (float)P;
}

// MEAN of fp16 rows (pc_mean_f16, src/pc_kern_f16.c:115-121): fp32 sum of the widened values, / P
__global__ void k_mean_f16(const uint16_t *__restrict__ x, long long x_ws, int P, int C, int ld, float *__restrict__ out,
                           long long o_ws) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x, win = blockIdx.y;
  if (c >= C) return;
  const uint16_t *xw = x + win * x_ws + c;
  float s = 0.f;
  for (int p = 0; p < P; p++) s = s + (float)hfrom(xw[(long long)p * ld]);
  out[win * o_ws + c] = s / (float)P;
}

// GEMV (bnn_gemv_f32 / bnn_gemv_h16, src/gemv.c:13-49) for WB windows per block: a thread owns one of the eight lane
// chains of one output (k = 8 i + l below K & ~7, then lanes 0..3 take the K & ~3 remainder), the eight lanes of an
// output are neighbours in a wave and meet by shuffles in the reference's pairwise order, lane 0 adds the scalar
// tail (product and sum rounded apart), the bias and the ReLU (v < 0 ? 0 : v). The windows' inputs sit in LDS; each
// weight read serves WB windows.
template <bool W16, int WB>
__global__ __launch_bounds__(256) void k_gemv(const void *__restrict__ wv, const float *__restrict__ bias, int N, int K,
                                              const float *__restrict__ x, long long x_ws, int act,
                                              float *__restrict__ out, long long o_ws, int B) {
  extern __shared__ float xs[];  // [WB][K]
  const int tid = threadIdx.x, l = tid & 7;
  const int win0 = blockIdx.y * WB, nw = B - win0 < WB ? B - win0 : WB;
  for (int i = tid; i < WB * K; i += 256) {
    const int wb = i / K, k = i - wb * K;
    xs[i] = wb < nw ? x[(win0 + wb) * x_ws + k] : 0.f;
  }
  __syncthreads();
  const int n = blockIdx.x * 32 + (tid >> 3);
  const int nn = n < N ? n : N - 1;  // lanes past N compute a valid row, store nothing
  const int K4 = K & ~3, K8 = K & ~7;
  auto wat = [&](int k) -> float {
    return W16 ? (float)hfrom(((const uint16_t *)wv)[(long long)nn * K + k]) : ((const float *)wv)[(long long)nn * K + k];
  };
  float a[WB];
#pragma unroll
  for (int wb = 0; wb < WB; wb++) a[wb] = 0.f;
#pragma unroll 4
  for (int k = l; k < K8; k += 8) {
    const float w = wat(k);
#pragma unroll
    for (int wb = 0; wb < WB; wb++) a[wb] = __builtin_fmaf(w, xs[wb * K + k], a[wb]);
  }
  if (l < 4 && K8 + l < K4) {
    const float w = wat(K8 + l);
#pragma unroll
    for (int wb = 0; wb < WB; wb++) a[wb] = __builtin_fmaf(w, xs[wb * K + K8 + l], a[wb]);
  }
#pragma unroll
  for (int wb = 0; wb < WB; wb++) {
    // lane l holds chain l: (c0 + c4) + (c1 + c5) and (c2 + c6) + (c3 + c7), then their sum
    const float p4 = __shfl_down(a[wb], 4, 8);       // lanes 0..3: chain l + 4
    const float s1 = a[wb] + p4;                       // lanes 0..3: c_l + c_{l+4}
    const float q1 = __shfl_down(s1, 1, 8);            // lane 0: c1 + c5; lane 2: c3 + c7
    const float s2 = s1 + q1;                          // lane 0: (c0+c4)+(c1+c5); lane 2: (c2+c6)+(c3+c7)
    const float q2 = __shfl_down(s2, 2, 8);
    float sum = s2 + q2;                               // lane 0: the pairwise total
    if (l == 0 && n < N && wb < nw) {
      for (int k = K4; k < K; k++) sum = sum + wat(k) * xs[wb * K + k];
      const float v = sum + bias[n];
      out[(win0 + wb) * o_ws + n] = act == 2 && v < 0.f ? 0.f : v;
    }
  }
}

// the device expf on its own (for its parity test against the C library)
__global__ void k_eval_expf(const float *__restrict__ x, float *__restrict__ y, long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = bnh_expf(x[i]);
}

// the device powf on its own (for its parity test against the C library)
__global__ void k_eval_powf(const float *__restrict__ x, const float *__restrict__ y, float *__restrict__ z,
                            long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) z[i] = bnh_powf(x[i], y[i]);
}

// ------------------------------------------------------------------ PAD: every element of the padded buffer
// PAD: a thread per V consecutive elements of one window's padded buffer (V = 16 bytes when the channel count, the
// row stride and the window strides allow, else 1), windows on grid.y; halo elements get zero
template <typename T, int V>
__global__ __launch_bounds__(256) void k_pad(const T *__restrict__ x, long long x_ws, int H, int W, int C, int ld,
                                             int h, T *__restrict__ xp, long long p_ws, int per) {
  const int i = (blockIdx.x * 256 + threadIdx.x) * V;
  if (i >= per) return;
  const long long win = blockIdx.y;
  const int Wp = W + 2 * h, px = i / C, c = i - px * C, y = px / Wp - h, xx = px - (px / Wp) * Wp - h;
  typedef T vt __attribute__((ext_vector_type(V)));
  vt v = (vt)0;
  if (y >= 0 && y < H && xx >= 0 && xx < W) v = *(const vt *)(x + win * x_ws + ((long long)y * W + xx) * ld + c);
  *(vt *)(xp + win * p_ws + i) = v;
}

// UNPAD (src/rt_ops_dot.c:109-128): the interior of a zero-haloed fp16 buffer [H+2][W+2][C] widened to fp32 rows
// [H][W][C]; a thread per 4 consecutive output elements of one window (W C % 4 == 0), windows on grid.y
__global__ __launch_bounds__(256) void k_unpad_f16(const uint16_t *__restrict__ x, long long x_ws, int H, int W, int C,
                                                   float *__restrict__ out, long long o_ws) {
  const int i = (blockIdx.x * 256 + threadIdx.x) * 4, row = W * C;
  if (i >= H * row) return;
  const long long win = blockIdx.y;
  const int y = i / row, r = i - y * row;
  const uint16_t *s = x + win * x_ws + ((long long)(y + 1) * (W + 2) + 1) * C + r;
  float4 v;
  v.x = (float)hfrom(s[0]);
  v.y = (float)hfrom(s[1]);
  v.z = (float)hfrom(s[2]);
  v.w = (float)hfrom(s[3]);
  *(float4 *)(out + win * o_ws + i) = v;
}

static int se_launch(const float *chsum, long long c_ws, int C, int rd, int P, const float *w1, const float *b1,
                     const float *w2t, const float *b2, float *gate, long long g_ws, float *work, void *D,
                     long long d_ws, int B, bool f16, void *stream, uint16_t *gh = nullptr, long long gh_ws = 0) {
  BNH_REQ(chsum && w1 && b1 && w2t && b2 && (gate || D) && B > 0);
  BNH_REQ(C > 0 && C % 4 == 0 && C <= 4096 && rd > 0 && rd <= 512 && P > 0);
  BNH_REQ(B == 1 || (c_ws >= C && (!gate || g_ws >= C) && (!D || d_ws >= (long long)P * C)));
  hipStream_t st = bnh_stream(stream);
  // with a gate buffer and C % 8 == 0 the gates go there first and a second kernel over every window's pixels
  // scales D (a block per group of windows scaling its own activations leaves most of the chip idle)
  const bool split = gate && D && C % 8 == 0;
  if (gate && work) {
    // the two FCs as kernels over all windows: fc1 into work [B][rd], fc2 + sigmoid into gate
    // windows per block: 4 (each weight read serves 4 windows) unless that leaves fewer than 512 blocks, then 2 or 1
    const long long rb1 = bnh_ceil_div(rd, 32);
    int wb1 = bnh_ceil_div(B, 4) * rb1 >= 512 ? 4 : bnh_ceil_div(B, 2) * rb1 >= 512 ? 2 : 1;
    if ((size_t)wb1 * C * 4 + (size_t)wb1 * 32 * 8 * 4 > 64 * 1024) wb1 = 1;
    const float inv = 1.f / (float)P;
    const dim3 g1((unsigned)bnh_ceil_div(B, wb1), (unsigned)rb1);
    const size_t l1 = sizeof(float) * ((size_t)wb1 * C + (size_t)wb1 * 32 * 8);
    if (wb1 == 4) hipLaunchKernelGGL((k_se_fc1<4>), g1, dim3(256), l1, st, chsum, c_ws, C, rd, inv, w1, b1, work, B);
    else if (wb1 == 2) hipLaunchKernelGGL((k_se_fc1<2>), g1, dim3(256), l1, st, chsum, c_ws, C, rd, inv, w1, b1, work, B);
    else hipLaunchKernelGGL((k_se_fc1<1>), g1, dim3(256), l1, st, chsum, c_ws, C, rd, inv, w1, b1, work, B);
    BNH_HIP(hipGetLastError());
    const long long cb2 = bnh_ceil_div(C, 256);
    const int wb2 = bnh_ceil_div(B, 4) * cb2 >= 512 ? 4 : bnh_ceil_div(B, 2) * cb2 >= 512 ? 2 : 1;
    const dim3 g2((unsigned)cb2, (unsigned)bnh_ceil_div(B, wb2));
    const size_t l2 = sizeof(float) * wb2 * (size_t)rd;
#define SE_FC2(W_, F_)                                                                                                 \
  hipLaunchKernelGGL((k_se_fc2<W_, F_>), g2, dim3(256), l2, st, work, C, rd, w2t, b2, gate, g_ws, B, gh, gh_ws)
    if (f16) { if (wb2 == 4) SE_FC2(4, true); else if (wb2 == 2) SE_FC2(2, true); else SE_FC2(1, true); }
    else { if (wb2 == 4) SE_FC2(4, false); else if (wb2 == 2) SE_FC2(2, false); else SE_FC2(1, false); }
#undef SE_FC2
    BNH_HIP(hipGetLastError());
    if (D && !split) {  // C % 8 != 0: the one-kernel form gates D (recomputing the same gates)
      work = nullptr;
    }
  }
  if (!(gate && work)) {
    // windows per block: as many as 64 KB of LDS holds, at most 4
    const size_t per = sizeof(float) * (2 * (size_t)C + 9 * (size_t)rd);
    int wg = (int)((64 * 1024) / per);
    wg = wg >= 4 ? 4 : wg >= 2 ? 2 : 1;
    if (wg > B) wg = B >= 4 ? 4 : B >= 2 ? 2 : 1;
    const dim3 grid((unsigned)bnh_ceil_div(B, wg));
    void *Dk = split ? nullptr : D;
#define SE_LAUNCH(W, F)                                                                                                \
  hipLaunchKernelGGL((k_se_f32<W, F>), grid, dim3(256), per * W, st, chsum, c_ws, C, rd, P, w1, b1, w2t, b2, gate,    \
                     g_ws, Dk, d_ws, B)
    if (f16) {
      if (wg == 4) SE_LAUNCH(4, true); else if (wg == 2) SE_LAUNCH(2, true); else SE_LAUNCH(1, true);
    } else {
      if (wg == 4) SE_LAUNCH(4, false); else if (wg == 2) SE_LAUNCH(2, false); else SE_LAUNCH(1, false);
    }
#undef SE_LAUNCH
    BNH_HIP(hipGetLastError());
  }
  if (!split) return 0;
  const long long n8 = (long long)P * C / 8;
  const unsigned esz = f16 ? 2 : 4;
  const bool vec = ((uintptr_t)D & 15) == 0 && ((uintptr_t)gate & 15) == 0 && g_ws % 4 == 0 &&
                   (d_ws * esz) % 16 == 0;
  const dim3 sg((unsigned)bnh_ceil_div(n8, 256), (unsigned)B);
  if (f16) {
    if (vec) hipLaunchKernelGGL((k_se_scale<true, true>), sg, dim3(256), 0, st, gate, g_ws, C, n8, D, d_ws);
    else hipLaunchKernelGGL((k_se_scale<true, false>), sg, dim3(256), 0, st, gate, g_ws, C, n8, D, d_ws);
  } else {
    if (vec) hipLaunchKernelGGL((k_se_scale<false, true>), sg, dim3(256), 0, st, gate, g_ws, C, n8, D, d_ws);
    else hipLaunchKernelGGL((k_se_scale<false, false>), sg, dim3(256), 0, st, gate, g_ws, C, n8, D, d_ws);
  }
  BNH_HIP(hipGetLastError());
  return 0;
}

extern "C" {

int bnh_zero_halo(void *xp, long long ws, int H, int W, int C, int h, int esz, int B, void *stream) {
  BNH_REQ(xp && H > 0 && W > 0 && C > 0 && h >= 0 && B > 0 && (esz == 4 || esz == 2));
  const long long per = (long long)(H + 2 * h) * (W + 2 * h) * C, total = 2LL * h * (W + 2 * h + H) * C * B;
  BNH_REQ(B == 1 || ws >= per);
  if (!h) return 0;
  const dim3 grid((unsigned)bnh_ceil_div(total, 256));
  if (esz == 4)
    hipLaunchKernelGGL(k_zero_halo<uint32_t>, grid, dim3(256), 0, bnh_stream(stream), (uint32_t *)xp, ws, H, W, C, h,
                       total);
  else
    hipLaunchKernelGGL(k_zero_halo<uint16_t>, grid, dim3(256), 0, bnh_stream(stream), (uint16_t *)xp, ws, H, W, C, h,
                       total);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_stem_f32(const float *img, long long i_ws, int H, int W, int k, int s, int Ho, int Wo, const float *w,
                 const float *bias, int Kp, int Np, int act, float *out, long long o_ws, int ldo, int opad, int B,
                 void *stream) {
  BNH_REQ(out && B > 0 && Ho > 0 && Wo > 0 && ldo > 0 && opad >= 0 && opad <= 3);
  BNH_REQ(B == 1 || o_ws >= (long long)(Ho + 2 * opad) * (Wo + 2 * opad) * ldo);
  if (opad && bnh_zero_halo(out, o_ws, Ho, Wo, ldo, opad, 4, B, stream)) return -1;
  return bnh_stem_f32_body(img, i_ws, H, W, k, s, Ho, Wo, w, bias, Kp, Np, act, out, o_ws, ldo, opad, B, stream);
}

int bnh_stem_f32_body(const float *img, long long i_ws, int H, int W, int k, int s, int Ho, int Wo, const float *w,
                      const float *bias, int Kp, int Np, int act, float *out, long long o_ws, int ldo, int opad, int B,
                      void *stream) {
  BNH_REQ(img && w && bias && out && B > 0 && k >= 1 && s >= 1 && Ho > 0 && Wo > 0);
  BNH_REQ((Ho - 1) * s + k <= H && (Wo - 1) * s + k <= W && Kp >= k * k && Kp % 4 == 0 && Np % 8 == 0);
  BNH_REQ(ldo >= Np && opad >= 0 && opad <= 3 && act >= 0 && act <= 2 && ldo % 4 == 0);
  BNH_REQ(((uintptr_t)w & 15) == 0 && ((uintptr_t)out & 3) == 0);
  BNH_REQ((long long)Np * (Kp + 1) * 4 <= 48 * 1024);  // the panels and the bias in LDS
  BNH_REQ(B == 1 || (i_ws >= (long long)H * W && o_ws >= (long long)(Ho + 2 * opad) * (Wo + 2 * opad) * ldo));
  const long long per = (long long)Ho * Wo * (Np / 4);
  BNH_REQ(per < (1LL << 31) && (long long)H * W < (1LL << 31));
  const bool vec = ((uintptr_t)out & 15) == 0 && (B == 1 || o_ws % 4 == 0);  // ldo % 4 == 0 already
  stem_launch<false>(dim3((unsigned)bnh_ceil_div(per, 256), (unsigned)B), bnh_stream(stream), vec, img, i_ws, W, k, s,
                     Ho, Wo, w, bias, Kp, Np, act, (void *)out, o_ws, ldo, opad, Np);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_stem_f32to16_body(const float *img, long long i_ws, int H, int W, int k, int s, int Ho, int Wo, const float *w,
                          const float *bias, int Kp, int N, int Np, int act, uint16_t *out, long long o_ws, int ldo,
                          int opad, int B, void *stream) {
  BNH_REQ(img && w && bias && out && B > 0 && k >= 1 && s >= 1 && Ho > 0 && Wo > 0 && N > 0 && N <= Np);
  BNH_REQ((Ho - 1) * s + k <= H && (Wo - 1) * s + k <= W && Kp >= k * k && Kp % 4 == 0 && Np % 8 == 0);
  BNH_REQ(ldo >= N && opad >= 0 && opad <= 3 && act >= 0 && act <= 2);
  BNH_REQ(((uintptr_t)w & 15) == 0);
  BNH_REQ((long long)Np * (Kp + 1) * 4 <= 48 * 1024);  // the panels and the bias in LDS
  BNH_REQ(B == 1 || (i_ws >= (long long)H * W && o_ws >= (long long)(Ho + 2 * opad) * (Wo + 2 * opad) * ldo));
  const long long per = (long long)Ho * Wo * (Np / 4);
  BNH_REQ(per < (1LL << 31) && (long long)H * W < (1LL << 31));
  const bool vec = ((uintptr_t)out & 7) == 0 && ldo % 4 == 0 && (B == 1 || o_ws % 4 == 0);
  stem_launch<true>(dim3((unsigned)bnh_ceil_div(per, 256), (unsigned)B), bnh_stream(stream), vec, img, i_ws, W, k, s,
                    Ho, Wo, w, bias, Kp, Np, act, (void *)out, o_ws, ldo, opad, N);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_stem_f32to16(const float *img, long long i_ws, int H, int W, int k, int s, int Ho, int Wo, const float *w,
                     const float *bias, int Kp, int N, int Np, int act, uint16_t *out, long long o_ws, int ldo, int opad,
                     int B, void *stream) {
  BNH_REQ(out && B > 0 && Ho > 0 && Wo > 0 && ldo > 0 && opad >= 0 && opad <= 3);
  BNH_REQ(B == 1 || o_ws >= (long long)(Ho + 2 * opad) * (Wo + 2 * opad) * ldo);
  if (opad && bnh_zero_halo(out, o_ws, Ho, Wo, ldo, opad, 2, B, stream)) return -1;
  return bnh_stem_f32to16_body(img, i_ws, H, W, k, s, Ho, Wo, w, bias, Kp, N, Np, act, out, o_ws, ldo, opad, B, stream);
}


int bnh_se_f32(const float *chsum, long long c_ws, int C, int rd, int P, const float *w1, const float *b1,
               const float *w2t, const float *b2, float *gate, long long g_ws, float *work, float *D, long long d_ws,
               int B, void *stream) {
  return se_launch(chsum, c_ws, C, rd, P, w1, b1, w2t, b2, gate, g_ws, work, D, d_ws, B, false, stream);
}

int bnh_se_f16(const float *chsum, long long c_ws, int C, int rd, int P, const float *w1, const float *b1,
               const float *w2t, const float *b2, float *gate, long long g_ws, float *work, uint16_t *D,
               long long d_ws, int B, void *stream) {
  BNH_REQ(D);
  return se_launch(chsum, c_ws, C, rd, P, w1, b1, w2t, b2, gate, g_ws, work, D, d_ws, B, true, stream);
}

int bnh_se_gate_f16(const float *chsum, long long c_ws, int C, int rd, int P, const float *w1, const float *b1,
                    const float *w2t, const float *b2, float *gate, long long g_ws, float *work, uint16_t *gh,
                    long long gh_ws, int B, void *stream) {
  BNH_REQ(gate && work && gh && C % 8 == 0 && (B == 1 || gh_ws >= C));
  return se_launch(chsum, c_ws, C, rd, P, w1, b1, w2t, b2, gate, g_ws, work, nullptr, 0, B, true, stream, gh, gh_ws);
}

int bnh_mean_f32(const float *x, long long x_ws, int P, int C, int ld, float *out, long long o_ws, int B,
                 void *stream) {
  BNH_REQ(x && out && P > 0 && C > 0 && ld >= C && B > 0);
  BNH_REQ(B == 1 || (x_ws >= (long long)P * ld && o_ws >= C));
  hipLaunchKernelGGL(k_mean_f32, dim3((unsigned)bnh_ceil_div(C, 64), (unsigned)B), dim3(64), 0, bnh_stream(stream), x,
                     x_ws, P, C, ld, out, o_ws);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_mean_f16(const uint16_t *x, long long x_ws, int P, int C, int ld, float *out, long long o_ws, int B,
                 void *stream) {
  BNH_REQ(x && out && P > 0 && C > 0 && ld >= C && B > 0);
  BNH_REQ(B == 1 || (x_ws >= (long long)P * ld && o_ws >= C));
  hipLaunchKernelGGL(k_mean_f16, dim3((unsigned)bnh_ceil_div(C, 64), (unsigned)B), dim3(64), 0, bnh_stream(stream), x,
                     x_ws, P, C, ld, out, o_ws);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_gemv(const void *w, int w16, const float *bias, int N, int K, const float *x, long long x_ws, int act,
             float *out, long long o_ws, int B, void *stream) {
  BNH_REQ(w && bias && x && out && N > 0 && K > 0 && B > 0 && (act == 0 || act == 2));
  BNH_REQ(B == 1 || (x_ws >= K && o_ws >= N));
  int wb = 8;
  while (wb > 1 && (size_t)wb * K * sizeof(float) > 64 * 1024) wb /= 2;
  BNH_REQ((size_t)K * sizeof(float) <= 64 * 1024);
  const dim3 grid((unsigned)bnh_ceil_div(N, 32), (unsigned)bnh_ceil_div(B, wb));
  const size_t lds = sizeof(float) * (size_t)wb * K;
  hipStream_t st = bnh_stream(stream);
#define GV(W, NB)                                                                                                      \
  hipLaunchKernelGGL((k_gemv<W, NB>), grid, dim3(256), lds, st, w, bias, N, K, x, x_ws, act, out, o_ws, B)
  if (w16) {
    if (wb == 8) GV(true, 8); else if (wb == 4) GV(true, 4); else if (wb == 2) GV(true, 2); else GV(true, 1);
  } else {
    if (wb == 8) GV(false, 8); else if (wb == 4) GV(false, 4); else if (wb == 2) GV(false, 2); else GV(false, 1);
  }
#undef GV
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_pad(const void *x, long long x_ws, int H, int W, int C, int ld, int h, int esz, void *xp, long long p_ws, int B,
            void *stream) {
  BNH_REQ(x && xp && H > 0 && W > 0 && C > 0 && ld >= C && h >= 0 && h <= 3 && B > 0 && (esz == 4 || esz == 2));
  const long long per = (long long)(H + 2 * h) * (W + 2 * h) * C;
  BNH_REQ(B == 1 || (x_ws >= (long long)H * W * ld && p_ws >= per));
  BNH_REQ(per < (1LL << 31));
  const int v = 16 / esz;  // elements per 16 bytes
  const bool vec = C % v == 0 && ld % v == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)xp & 15) == 0 &&
                   (B == 1 || (x_ws % v == 0 && p_ws % v == 0));
  const dim3 grid((unsigned)bnh_ceil_div(per, 256LL * (vec ? v : 1)), (unsigned)B);
  hipStream_t st = bnh_stream(stream);
  if (esz == 4) {
    if (vec) hipLaunchKernelGGL((k_pad<uint32_t, 4>), grid, dim3(256), 0, st, (const uint32_t *)x, x_ws, H, W, C, ld, h,
                                (uint32_t *)xp, p_ws, (int)per);
    else hipLaunchKernelGGL((k_pad<uint32_t, 1>), grid, dim3(256), 0, st, (const uint32_t *)x, x_ws, H, W, C, ld, h,
                            (uint32_t *)xp, p_ws, (int)per);
  } else {
    if (vec) hipLaunchKernelGGL((k_pad<uint16_t, 8>), grid, dim3(256), 0, st, (const uint16_t *)x, x_ws, H, W, C, ld, h,
                                (uint16_t *)xp, p_ws, (int)per);
    else hipLaunchKernelGGL((k_pad<uint16_t, 1>), grid, dim3(256), 0, st, (const uint16_t *)x, x_ws, H, W, C, ld, h,
                            (uint16_t *)xp, p_ws, (int)per);
  }
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_unpad_f16(const uint16_t *x, long long x_ws, int H, int W, int C, float *out, long long o_ws, int B,
                  void *stream) {
  BNH_REQ(x && out && H > 0 && W > 0 && C > 0 && (W * C) % 4 == 0 && B > 0);
  BNH_REQ(((uintptr_t)out & 15) == 0 && (B == 1 || (x_ws >= (long long)(H + 2) * (W + 2) * C &&
                                                    o_ws >= (long long)H * W * C && o_ws % 4 == 0)));
  BNH_REQ((long long)H * W * C < (1LL << 31));
  const dim3 grid((unsigned)bnh_ceil_div((long long)H * W * C, 1024), (unsigned)B);
  hipLaunchKernelGGL(k_unpad_f16, grid, dim3(256), 0, bnh_stream(stream), x, x_ws, H, W, C, out, o_ws);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_eval_powf(const float *x, const float *y, float *z, long long n, void *stream) {
  BNH_REQ(x && y && z && n >= 0);
  if (!n) return 0;
  hipLaunchKernelGGL(k_eval_powf, dim3((unsigned)bnh_ceil_div(n, 256)), dim3(256), 0, bnh_stream(stream), x, y, z, n);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_eval_expf(const float *x, float *y, long long n, void *stream) {
  BNH_REQ(x && y && n >= 0);
  if (!n) return 0;
  hipLaunchKernelGGL(k_eval_expf, dim3((unsigned)bnh_ceil_div(n, 256)), dim3(256), 0, bnh_stream(stream), x, y, n);
  BNH_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
