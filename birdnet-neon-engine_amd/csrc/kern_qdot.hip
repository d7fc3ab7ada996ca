// The dotprod family's int8 arithmetic (src/gemm_s8.c, src/rt_ops_dot.c:173-585), bit-identical to the reference:
//   - activation rows quantised to [-128, 127] with a per-row (or per-tensor) scale and a float zero point
//     (quant_rows_f32 / quant_rows_f16 / quant_tensor_pad_f32), weights per channel to [-127, 127] (qw_pack);
//   - exact int32 sums on int8 MFMA, then v = (b + (f sw) sa) + swsum (sa zp), both sums fused, and the fp16 (table
//     SiLU) or fp32 (silu_f32_a, ReLU, residual) store;
//   - the 3 x 3 conv as an implicit im2col over the quantised zero-point-haloed copy;
//   - the SED heads (axis means, max + average pools, fc / att / cla GEMMs, clipped soft-max), the fp16-weight SE gate
//     and the generalised mean.
// MFMA i8 16x16x64 tiles: lane l holds 16 k bytes (chunk l >> 4) of row / channel l & 15; accumulator r of lane l is
// row 4 (l >> 4) + r, channel l & 15.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "bnh_expf.h"
#include "bnh_f16.h"
#include "bnh_internal.h"
#include "bnh_powf.h"
#include "bnh_num.h"

typedef int v4i __attribute__((ext_vector_type(4)));

struct bnh_qdw {
  int N, K, Kp, Np;  // Np: N rounded up to 16 (zero channels past N); Kp: K rounded up to 16
  int8_t *w;         // [Np][Kp], zero past K
  float *scale, *swsum, *bias;
};

// ------------------------------------------------------------------ shared arithmetic
// params (src/gemm_s8.c:295-304)
BNH_DEV void qd_params(float mn, float mx, float &s, float &zp, float &inv) {
  mn = bnh_fminnm(mn, 0.f);
  mx = bnh_fmaxnm(mx, 0.f);
  const float d = mx - mn;
  s = d > 0.f ? d / 255.f : 1.f;
  inv = 1.f / s;
  zp = __builtin_rintf(mn * inv) + 128.f;
}
BNH_DEV int8_t qd_clamp8(int32_t q) { return (int8_t)(q > 127 ? 127 : (q < -128 ? -128 : q)); }
// q8_f32x8 lane (src/gemm_s8.c:284-293): fma(x, inv, 1.5 * 2^23) holds rint(x inv) in its low mantissa bits
BNH_DEV int8_t qd_magic(float x, float inv, int32_t zofs) {
  return qd_clamp8((int32_t)(bnh_bits(__builtin_fmaf(x, inv, 12582912.0f)) - (uint32_t)zofs));
}
// the scalar tails: rint(v) - zp in fp32, clamped
BNH_DEV int8_t qd_tail(float v, float zp) {
  const float q = __builtin_rintf(v) - zp;
  return (int8_t)(q > 127.f ? 127 : (q < -128.f ? -128 : (int)q));
}
// exp2_p5_f32 lane (src/act.h:9-21)
BNH_DEV float qd_exp2_p5(float t) {
  const float magic = 12582912.0f;
  const float tm = t + magic, n = tm - magic, f = t - n;
  const uint32_t ni = bnh_bits(tm) << 23;
  float p = __builtin_fmaf(1.3333558e-3f, f, 9.6181291e-3f);
  p = __builtin_fmaf(p, f, 5.5504109e-2f);
  p = __builtin_fmaf(p, f, 2.4022651e-1f);
  p = __builtin_fmaf(p, f, 6.9314718e-1f);
  p = __builtin_fmaf(p, f, 1.0f);
  return bnh_float(bnh_bits(p) + ni);
}
// 1 / (1 + 2^t), t clamped to [-126, 126]: FRECPE and two Newton steps (silu_f32_a src/act.h:41-49, the SE gate's
// sigmoid src/rt_ops_dot.c:409-416)
BNH_DEV float qd_rcp1p_exp2(float t) {
  t = bnh_fmin(bnh_fmax(t, -126.f), 126.f);
  const float d = qd_exp2_p5(t) + 1.0f;
  float r = bnh_frecpe(d);
  r = r * bnh_frecps(d, r);
  r = r * bnh_frecps(d, r);
  return r;
}
BNH_DEV float qd_silu_f32_a(float x) { return x * qd_rcp1p_exp2(x * -1.44269504f); }
// log2_f32 lane (src/act.h:23-38)
BNH_DEV float qd_log2(float x) {
  const int32_t xi = (int32_t)bnh_bits(x);
  const int32_t e = (int32_t)((uint32_t)xi - 0x3F3504F3u) >> 23;
  const float mnt = bnh_float((uint32_t)xi - ((uint32_t)e << 23));
  const float z = mnt - 1.0f;
  const float u = z / (mnt + 1.0f);
  const float u2 = u * u;
  float pp = __builtin_fmaf(u2, 1.f / 9, 1.f / 7);
  pp = __builtin_fmaf(pp, u2, 1.f / 5);
  pp = __builtin_fmaf(pp, u2, 1.f / 3);
  pp = __builtin_fmaf(pp, u2, 1.f);
  const float ln = (u * 2.f) * pp;
  return __builtin_fmaf(ln, 1.44269504f, (float)e);
}
BNH_DEV float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = bnh_fmin(v, __shfl_xor(v, o));
  return v;
}
BNH_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = bnh_fmax(v, __shfl_xor(v, o));
  return v;
}

// ------------------------------------------------------------------ per-row quantisation
// One wavefront per row (rows = B * M, window w = row / M). The range: FMIN / FMAX from 0 over k < K & ~3 (fp32) or
// over the (gated, fp16-rounded) k < K & ~7 (fp16) in any order (NaN-propagating minima do not depend on it), then
// the tail in order with FMINNM / FMAXNM. The codes: 4 per lane per pass, one 32-bit store each (Kp % 16 == 0).
template <bool F16>
__global__ __launch_bounds__(256) void k_qd_quant(const void *__restrict__ xv, long long x_ws, int ldx, int M,
                                                  double rM, int K, int Kp, const uint16_t *__restrict__ gate,
                                                  long long g_ws, int8_t *__restrict__ a, long long a_ws,
                                                  float *__restrict__ rq, long long rq_ws, long long rows) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int w = bnh_div(row, M, rM), m = (int)(row - (long long)w * M);
  int8_t *o = a + w * a_ws + (long long)m * Kp;
  const float *r32 = F16 ? nullptr : (const float *)xv + w * x_ws + (long long)m * ldx;
  const uint16_t *r16 = F16 ? (const uint16_t *)xv + w * x_ws + (long long)m * ldx : nullptr;
  const uint16_t *g = F16 && gate ? gate + w * g_ws : nullptr;
  float mn, mx;
  int kt;
  if (F16) {
    kt = K & ~7;
    h16 hn = (h16)0, hx = (h16)0;
    for (int c = lane; c < kt; c += 64) {
      h16 h = hfrom(r16[c]);
      if (g) h = h * hfrom(g[c]);
      hn = hmin(hn, h);
      hx = hmax(hx, h);
    }
    mn = wave_min((float)hn);
    mx = wave_max((float)hx);
  } else {
    kt = K & ~3;
    mn = 0.f;
    mx = 0.f;
    for (int c = lane; c < kt; c += 64) {
      const float v = r32[c];
      mn = bnh_fmin(mn, v);
      mx = bnh_fmax(mx, v);
    }
    mn = wave_min(mn);
    mx = wave_max(mx);
  }
  for (int c = kt; c < K; c++) {
    const float v = F16 ? (float)hfrom(r16[c]) * (g ? (float)hfrom(g[c]) : 1.f) : r32[c];
    mn = bnh_fminnm(mn, v);
    mx = bnh_fmaxnm(mx, v);
  }
  float s, zp, inv;
  qd_params(mn, mx, s, zp, inv);
  if (lane == 0) {
    rq[w * rq_ws + 2 * m] = s;
    rq[w * rq_ws + 2 * m + 1] = zp;
  }
  const int32_t zofs = 0x4B400000 + (int32_t)zp;
  const h16 hinv = f2h(inv);
  const uint16_t zo = (uint16_t)(0x6600 + (int)zp);
  const int kq = F16 ? K & ~15 : K & ~7;  // codes by the vector form below kq, the scalar tail above
  for (int c0 = 4 * lane; c0 < Kp; c0 += 256) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = c0 + i;
      int8_t q = 0;
      if (c < kq) {
        if (F16) {
          h16 h = hfrom(r16[c]);
          if (g) h = h * hfrom(g[c]);
          q = qd_clamp8((int16_t)(uint16_t)(hbits(hfma(h, hinv, (h16)1536.0f)) - zo));
        } else {
          q = qd_magic(r32[c], inv, zofs);
        }
      } else if (c < K) {
        const float v = F16 ? (float)hfrom(r16[c]) * (g ? (float)hfrom(g[c]) : 1.f) : r32[c];
        q = qd_tail(v * inv, zp);
      }
      word |= (uint32_t)(uint8_t)q << (8 * i);
    }
    *(uint32_t *)(o + c0) = word;
  }
}

// The same with L lanes per row (64 / L rows per wavefront) and 8 channels per lane per pass: 16-byte loads (fp16)
// or two 16-byte loads (fp32), one 8-byte store of codes. K % 8 == 0, so every 8-channel chunk lies wholly in the
// range part and wholly in the fp16 (or magic-number) code part or in the fp32 tail part; the lane group's range
// reduction is order-free (NaN-propagating minima).
typedef _Float16 qv8h __attribute__((ext_vector_type(8)));
template <int L, bool F16>
__global__ __launch_bounds__(256) void k_qd_quant_v(const void *__restrict__ xv, long long x_ws, int ldx, int M,
                                                    double rM, int K, int Kp, const uint16_t *__restrict__ gate,
                                                    long long g_ws, int8_t *__restrict__ a, long long a_ws,
                                                    float *__restrict__ rq, long long rq_ws, long long rows) {
  const int lane = threadIdx.x & 63, sub = lane % L;
  long long row = ((long long)blockIdx.x * 256 + threadIdx.x) / L;
  const bool live = row < rows;
  if (!live) row = rows - 1;  // a valid row: the group's lanes take part in the shuffles, nothing is stored
  const int w = bnh_div(row, M, rM), m = (int)(row - (long long)w * M);
  int8_t *o = a + w * a_ws + (long long)m * Kp;
  const float *r32 = F16 ? nullptr : (const float *)xv + w * x_ws + (long long)m * ldx;
  const _Float16 *r16 = F16 ? (const _Float16 *)xv + w * x_ws + (long long)m * ldx : nullptr;
  const _Float16 *g = F16 && gate ? (const _Float16 *)gate + w * g_ws : nullptr;
  float mn = 0.f, mx = 0.f;
  for (int c0 = 8 * sub; c0 < K; c0 += 8 * L) {
    if (F16) {
      qv8h h = *(const qv8h *)(r16 + c0);
      if (g) h = h * *(const qv8h *)(g + c0);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        mn = bnh_fmin(mn, (float)h[i]);
        mx = bnh_fmax(mx, (float)h[i]);
      }
    } else {
      const float4 u = *(const float4 *)(r32 + c0), v = *(const float4 *)(r32 + c0 + 4);
      const float e[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        mn = bnh_fmin(mn, e[i]);
        mx = bnh_fmax(mx, e[i]);
      }
    }
  }
#pragma unroll
  for (int off = 1; off < L; off <<= 1) {
    mn = bnh_fmin(mn, __shfl_xor(mn, off));
    mx = bnh_fmax(mx, __shfl_xor(mx, off));
  }
  float s, zp, inv;
  qd_params(mn, mx, s, zp, inv);
  if (live && sub == 0) {
    rq[w * rq_ws + 2 * m] = s;
    rq[w * rq_ws + 2 * m + 1] = zp;
  }
  if (!live) return;
  const int32_t zofs = 0x4B400000 + (int32_t)zp;
  const h16 hinv = f2h(inv);
  const uint16_t zo = (uint16_t)(0x6600 + (int)zp);
  const int kq = F16 ? K & ~15 : K;  // fp16 codes below kq, the fp32 tail from there (the fp32 rows: magic codes)
  for (int c0 = 8 * sub; c0 < Kp; c0 += 8 * L) {
    uint32_t lo = 0, hi = 0;
    if (c0 < K) {
      if (F16) {
        const qv8h xr = *(const qv8h *)(r16 + c0);
        const qv8h gr = g ? *(const qv8h *)(g + c0) : (qv8h){};
        if (c0 < kq) {
          const qv8h h = g ? xr * gr : xr;  // the gated product rounded to fp16
#pragma unroll
          for (int i = 0; i < 8; i++)
            (i < 4 ? lo : hi) |= (uint32_t)(uint8_t)qd_clamp8((int16_t)(uint16_t)(hbits(hfma(h[i], hinv, (h16)1536.0f)) -
                                                                                    zo)) << (8 * (i & 3));
        } else {  // the fp32 tail: the unrounded product (exact in fp32), times the fp32 inv
#pragma unroll
          for (int i = 0; i < 8; i++) {
            const float v = (float)xr[i] * (g ? (float)gr[i] : 1.f);
            (i < 4 ? lo : hi) |= (uint32_t)(uint8_t)qd_tail(v * inv, zp) << (8 * (i & 3));
          }
        }
      } else {
        const float4 u = *(const float4 *)(r32 + c0), v = *(const float4 *)(r32 + c0 + 4);
        const float e[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 8; i++) (i < 4 ? lo : hi) |= (uint32_t)(uint8_t)qd_magic(e[i], inv, zofs) << (8 * (i & 3));
      }
    }
    *(uint2 *)(o + c0) = make_uint2(lo, hi);
  }
}

// ------------------------------------------------------------------ GEMM + fp32 FMA epilogue
struct QdEpi {
  int act;          // 0 none, 1 SiLU, 2 ReLU
  int out_f16;      // 1: fp16 out (act 0 / 1), 0: fp32 out (+ residual)
  void *out;
  long long out_ws;
  int ldo, ow, opad;
  double r_ow;
  const float *res;  // fp32 rows [M][ldo]
  long long res_ws;
};
BNH_DEV long long epi_row(int m, const QdEpi &e) {  // the (zero-haloed) output row of pixel m
  if (!e.opad) return m;
  const int y = bnh_div(m, e.ow, e.r_ow);
  return (long long)(y + e.opad) * (e.ow + 2 * e.opad) + (m - y * e.ow) + e.opad;
}
struct QdConv {  // the 3 x 3 implicit im2col: A row m = output pixel (m / Wo, m % Wo) of the haloed int8 copy
  int C, s, pt, pl, Wo, Wp;
  double r_wo;
};

// A block owns 128 rows; each wave 32 of them (2 MFMA row tiles) across the 64-channel groups [g0, g1) of its part.
// CONV: k = 3 C ky + (kx C + c) over the haloed copy (its rows hold the 3 C bytes of kx = 0..2 contiguously), each
// 16-byte chunk as two 8-byte halves, zero past 9 C.
// VEC: each wave's 16 x 64 tile leaves the accumulators through LDS after its epilogue (the same operations, the
// fp16 SiLU two values at a time from an LDS table) and is stored as 16-byte row chunks (fp32: the residual chunk
// added to each), instead of one 2- or 4-byte store per value.
template <bool CONV, bool VEC>
__global__ __launch_bounds__(256) void k_qd_gemm(const int8_t *__restrict__ a, long long a_ws, int lda,
                                                 const float *__restrict__ rq, long long rq_ws, int per_tensor, int M,
                                                 double rM, long long rows, const int8_t *__restrict__ wt,
                                                 const float *__restrict__ sw, const float *__restrict__ sws,
                                                 const float *__restrict__ bias, int Kp, int Np, int gsplit, QdEpi e,
                                                 QdConv cv) {
  constexpr int RB = 128, TS = 68;  // TS: the tile's LDS row stride in floats (64 channels + 4)
  __shared__ long long s_a[RB], s_o[RB], s_r[RB];
  __shared__ __attribute__((aligned(16))) float s_t[VEC ? 4 : 1][VEC ? 16 * TS : 1];
  __shared__ uint32_t s_t01[16];
  __shared__ uint16_t s_t2[16];
  if (threadIdx.x < 16) {
    s_t01[threadIdx.x] = (uint32_t)k_silu_c0[threadIdx.x] | ((uint32_t)k_silu_c1[threadIdx.x] << 16);
    s_t2[threadIdx.x] = k_silu_c2[threadIdx.x];
  }
  __shared__ float s_sa[RB], s_zs[RB];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const unsigned lb = gsplit > 1 ? bnh_xcd_block(blockIdx.x, gridDim.x) : blockIdx.x;
  const long long rowB = (long long)(lb / gsplit) * RB;
  const int ng = (Np + 63) / 64, part = (int)(lb % gsplit);
  const int g0 = part * ng / gsplit, g1 = (part + 1) * ng / gsplit;
  for (int i = threadIdx.x; i < RB; i += 256) {
    const long long row = rowB + i < rows ? rowB + i : rows - 1;  // rows past the end repeat the last row
    const int w = bnh_div(row, M, rM), m = (int)(row - (long long)w * M);
    if (CONV) {
      const int oy = bnh_div(m, cv.Wo, cv.r_wo), ox = m - oy * cv.Wo;
      s_a[i] = w * a_ws + ((long long)(oy * cv.s - cv.pt + 1) * cv.Wp + (ox * cv.s - cv.pl + 1)) * cv.C;
    } else {
      s_a[i] = w * a_ws + (long long)m * lda;
    }
    s_o[i] = w * e.out_ws + epi_row(m, e) * e.ldo;
    s_r[i] = e.res ? w * e.res_ws + (long long)m * e.ldo : 0;
    const float *q = rq + w * rq_ws + (per_tensor ? 0 : 2 * m);
    s_sa[i] = q[0];
    s_zs[i] = q[0] * q[1];
  }
  __syncthreads();
  const int lr0 = wave * 32;
  if (rowB + lr0 >= rows) return;
  const int kc = (lane >> 4) * 16;
  const long long ab[2] = {s_a[lr0 + (lane & 15)], s_a[lr0 + 16 + (lane & 15)]};
  const int C3 = 3 * cv.C, K9 = 9 * cv.C, rowb = cv.Wp * cv.C;
  for (int g = g0; g < g1; g++) {
    const int n0 = 64 * g;
    const int jn = Np - n0 >= 64 ? 4 : (Np - n0) / 16;  // Np % 16 == 0
    const int8_t *bp = wt + (long long)(n0 + (lane & 15)) * Kp + kc;
    v4i acc[2][4];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[t][j] = (v4i){0, 0, 0, 0};
    for (int k0 = 0; k0 < Kp; k0 += 64) {
      const int k = k0 + kc;
      const bool kin = k < Kp;
      v4i av[2], bv[4];
#pragma unroll
      for (int t = 0; t < 2; t++) {
        if (CONV) {
          uint2 h[2];
#pragma unroll
          for (int hh = 0; hh < 2; hh++) {
            const int kk = k + 8 * hh;
            h[hh] = make_uint2(0u, 0u);
            if (kk < K9) {
              const int ky = (kk >= C3) + (kk >= 2 * C3);
              h[hh] = *(const uint2 *)(a + ab[t] + (long long)ky * rowb + (kk - ky * C3));
            }
          }
          av[t] = (v4i){(int)h[0].x, (int)h[0].y, (int)h[1].x, (int)h[1].y};
        } else {
          av[t] = kin ? *(const v4i *)(a + ab[t] + k) : (v4i){0, 0, 0, 0};
        }
      }
#pragma unroll
      for (int j = 0; j < 4; j++) bv[j] = kin && j < jn ? *(const v4i *)(bp + (long long)16 * j * Kp + k0) : (v4i){0, 0, 0, 0};
#pragma unroll
      for (int t = 0; t < 2; t++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          if (j < jn) acc[t][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[t], bv[j], acc[t][j], 0, 0, 0);
    }
    // epilogue (tile_row / affine4, src/gemm_s8.c:54-87,143-150)
    float swn[4], ssn[4], bn[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + 16 * j + (lane & 15);
      const bool ok = j < jn;
      swn[j] = ok ? sw[n] : 0.f;
      ssn[j] = ok ? sws[n] : 0.f;
      bn[j] = ok ? bias[n] : 0.f;
    }
    if (VEC) {
      float *T = s_t[wave];
      const int nv = Np - n0 < 64 ? Np - n0 : 64;  // channels of this group (a multiple of 16)
#pragma unroll
      for (int t = 0; t < 2; t++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          if (j >= jn) break;
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int lr = lr0 + 16 * t + 4 * (lane >> 4) + r;
            const float f = (float)acc[t][j][r];
            const float v0 = f * swn[j];
            v[r] = __builtin_fmaf(ssn[j], s_zs[lr], __builtin_fmaf(v0, s_sa[lr], bn[j]));
          }
          const int col = 16 * j + (lane & 15), rb = 4 * (lane >> 4);
          if (e.out_f16) {
            uint16_t *Th = (uint16_t *)T;  // [16][2 TS] halves
#pragma unroll
            for (int r = 0; r < 4; r += 2) {
              h2 hv = (h2){f2h(v[r]), f2h(v[r + 1])};
              if (e.act == 1) hv = silu2_lut(hv, s_t01, s_t2);
              Th[(rb + r) * 2 * TS + col] = hbits(hv[0]);
              Th[(rb + r + 1) * 2 * TS + col] = hbits(hv[1]);
            }
          } else {
#pragma unroll
            for (int r = 0; r < 4; r++) {
              float y = v[r];
              if (e.act == 1) y = qd_silu_f32_a(y);
              else if (e.act == 2) y = bnh_relu_f32(y);
              T[(rb + r) * TS + col] = y;
            }
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (e.out_f16) {  // 16 rows x 8 chunks of 8 halves: two per lane
#pragma unroll
          for (int it = 0; it < 2; it++) {
            const int rr = 8 * it + (lane >> 3), ch = lane & 7, lr = lr0 + 16 * t + rr;
            if (8 * ch < nv && rowB + lr < rows)
              *(uint4 *)((uint16_t *)e.out + s_o[lr] + n0 + 8 * ch) =
                  *(const uint4 *)((const uint16_t *)T + rr * 2 * TS + 8 * ch);
          }
        } else {  // 16 rows x 16 chunks of 4 floats: four per lane, the residual chunks loaded first
          float4 rv4[4];
#pragma unroll
          for (int it = 0; it < 4; it++) {
            const int rr = 4 * it + (lane >> 4), ch = lane & 15, lr = lr0 + 16 * t + rr;
            rv4[it] = e.res && 4 * ch < nv && rowB + lr < rows ? *(const float4 *)(e.res + s_r[lr] + n0 + 4 * ch)
                                                              : make_float4(0.f, 0.f, 0.f, 0.f);
          }
#pragma unroll
          for (int it = 0; it < 4; it++) {
            const int rr = 4 * it + (lane >> 4), ch = lane & 15, lr = lr0 + 16 * t + rr;
            if (4 * ch < nv && rowB + lr < rows) {
              float4 y = *(const float4 *)(T + rr * TS + 4 * ch);
              if (e.res) {
                y.x = y.x + rv4[it].x;
                y.y = y.y + rv4[it].y;
                y.z = y.z + rv4[it].z;
                y.w = y.w + rv4[it].w;
              }
              *(float4 *)((float *)e.out + s_o[lr] + n0 + 4 * ch) = y;
            }
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
      continue;
    }
#pragma unroll
    for (int t = 0; t < 2; t++) {
      float rv[4][4];
      if (e.res) {  // residuals of the tile first (out and res may alias)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int lr = lr0 + 16 * t + 4 * (lane >> 4) + r;
#pragma unroll
          for (int j = 0; j < 4; j++)
            rv[r][j] = j < jn && rowB + lr < rows ? e.res[s_r[lr] + n0 + 16 * j + (lane & 15)] : 0.f;
        }
      }
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int lr = lr0 + 16 * t + 4 * (lane >> 4) + r;
        if (rowB + lr >= rows) continue;
        const float sa = s_sa[lr], zs = s_zs[lr];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          if (j >= jn) break;
          const int n = n0 + 16 * j + (lane & 15);
          const float f = (float)acc[t][j][r];
          const float v0 = f * swn[j];
          const float v = __builtin_fmaf(ssn[j], zs, __builtin_fmaf(v0, sa, bn[j]));
          if (e.out_f16) {
            h16 h = f2h(v);
            if (e.act == 1) h = silu_lut_h(h);
            ((uint16_t *)e.out)[s_o[lr] + n] = hbits(h);
          } else {
            float y = v;
            if (e.act == 1) y = qd_silu_f32_a(y);
            else if (e.act == 2) y = bnh_relu_f32(y);
            if (e.res) y = y + rv[r][j];
            ((float *)e.out)[s_o[lr] + n] = y;
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------------ per-tensor quantisation into a haloed copy
// quant_tensor_pad_f32 (src/gemm_s8.c:373-396). Pass 1: the partial minima / maxima of nbk slices of each window's
// H W C values (FMIN / FMAX from 0). Pass 2: every block folds its window's partials (the same result whatever the
// order), derives (scale, zp) and writes its slice of the (H + 2) x (W + 2) x C copy, 4 codes per thread per pass:
// the halo holds -zp, the interior the magic-number codes. Block 0 of a window stores rq.
__global__ __launch_bounds__(256) void k_qd_tminmax(const float *__restrict__ x, long long x_ws, long long n, int nbk,
                                                    float *__restrict__ part, long long p_ws) {
  __shared__ float s_mn[4], s_mx[4];
  const int w = blockIdx.y;
  const float *xw = x + w * x_ws;
  const long long i0 = n * blockIdx.x / nbk, i1 = n * (blockIdx.x + 1) / nbk;
  float mn = 0.f, mx = 0.f;
  for (long long i = i0 + threadIdx.x; i < i1; i += 256) {
    const float v = xw[i];
    mn = bnh_fmin(mn, v);
    mx = bnh_fmax(mx, v);
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) {
    s_mn[threadIdx.x >> 6] = mn;
    s_mx[threadIdx.x >> 6] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    part[w * p_ws + 2 * blockIdx.x] = bnh_fmin(bnh_fmin(s_mn[0], s_mn[1]), bnh_fmin(s_mn[2], s_mn[3]));
    part[w * p_ws + 2 * blockIdx.x + 1] = bnh_fmax(bnh_fmax(s_mx[0], s_mx[1]), bnh_fmax(s_mx[2], s_mx[3]));
  }
}
__global__ __launch_bounds__(256) void k_qd_tquant(const float *__restrict__ x, long long x_ws, int H, int W, int C,
                                                   const float *__restrict__ part, long long p_ws, int nbk,
                                                   int8_t *__restrict__ xp,
                                                   long long xp_ws, float *__restrict__ rq, long long rq_ws,
                                                   int nbq) {
  __shared__ float s_mn[4], s_mx[4];
  const int w = blockIdx.y;
  float mn = 0.f, mx = 0.f;
  for (int i = threadIdx.x; i < nbk; i += 256) {
    mn = bnh_fmin(mn, part[w * p_ws + 2 * i]);
    mx = bnh_fmax(mx, part[w * p_ws + 2 * i + 1]);
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) {
    s_mn[threadIdx.x >> 6] = mn;
    s_mx[threadIdx.x >> 6] = mx;
  }
  __syncthreads();
  mn = bnh_fmin(bnh_fmin(s_mn[0], s_mn[1]), bnh_fmin(s_mn[2], s_mn[3]));
  mx = bnh_fmax(bnh_fmax(s_mx[0], s_mx[1]), bnh_fmax(s_mx[2], s_mx[3]));
  float s, zp, inv;
  qd_params(mn, mx, s, zp, inv);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    rq[w * rq_ws] = s;
    rq[w * rq_ws + 1] = zp;
  }
  const int32_t zofs = 0x4B400000 + (int32_t)zp;
  const uint32_t halo = (uint32_t)(uint8_t)(int8_t)(-(int)zp) * 0x01010101u;
  const int Wp = W + 2;
  const long long nq = (long long)(H + 2) * Wp * C / 4;  // 4-byte groups (C % 4 == 0: a group is in one pixel)
  const long long q0 = nq * blockIdx.x / nbq, q1 = nq * (blockIdx.x + 1) / nbq;
  const float *xw = x + w * x_ws;
  uint32_t *ow = (uint32_t *)(xp + w * xp_ws);
  for (long long gi = q0 + threadIdx.x; gi < q1; gi += 256) {
    const long long byte = 4 * gi, pix = byte / C;
    const int c = (int)(byte - pix * C), y = (int)(pix / Wp), xx = (int)(pix - (long long)y * Wp);
    uint32_t word = halo;
    if (y >= 1 && y <= H && xx >= 1 && xx <= W) {
      const float *src = xw + ((long long)(y - 1) * W + (xx - 1)) * C + c;
      word = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) word |= (uint32_t)(uint8_t)qd_magic(src[i], inv, zofs) << (8 * i);
    }
    ow[gi] = word;
  }
}

// ------------------------------------------------------------------ SED heads (HEADS_S8, src/rt_ops_dot.c:520-572)
// s[t][c]: the mean over the other axis (AX 0: row t of W pixels, AX 1: column t of H pixels), one sequential sum
// from 0 per output, / the count
template <int AX>
__global__ __launch_bounds__(256) void k_hd_means(const float *__restrict__ F, long long f_ws, int H, int W, int C,
                                                  float *__restrict__ s, long long s_ws) {
  const int w = blockIdx.y, Lt = AX == 0 ? H : W;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= Lt * C) return;
  const int t = i / C, ch = i - t * C;
  const float *Fw = F + w * f_ws;
  float a2 = 0.f;
  if (AX == 0) {
    for (int u = 0; u < W; u++) a2 += Fw[(long long)(t * W + u) * C + ch];
    s[w * s_ws + i] = a2 / (float)W;
  } else {
    for (int u = 0; u < H; u++) a2 += Fw[(long long)(u * W + t) * C + ch];
    s[w * s_ws + i] = a2 / (float)H;
  }
}
// pooled[t][c] = max over the (up to) 3 neighbours (FMAXNM from -FLT_MAX) + their sum of v * 0.33333334 in order
__global__ __launch_bounds__(256) void k_hd_pool(const float *__restrict__ s, long long s_ws, int Lt, int C,
                                                 float *__restrict__ pooled, long long p_ws) {
  const int w = blockIdx.y;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= Lt * C) return;
  const int t = i / C, ch = i - t * C;
  const float *sw = s + w * s_ws;
  float mx = -3.402823466e38f, sum = 0.f;
  for (int d = -1; d <= 1; d++) {
    const int u = t + d;
    if (u < 0 || u >= Lt) continue;
    const float v = sw[u * C + ch];
    mx = bnh_fmaxnm(mx, v);
    sum += v * 0.33333334f;
  }
  pooled[w * p_ws + i] = mx + sum;
}
// per class k < nc: att clipped to [-10, 10], soft-max over t (the C library's expf), logits[k] += sum(ev cla) / z
__global__ __launch_bounds__(256) void k_hd_softmax(const float *__restrict__ att, const float *__restrict__ cla,
                                                    long long a_ws, int Lt, int ncp, int nc, float *__restrict__ logits,
                                                    long long l_ws) {
  const int w = blockIdx.y, k = blockIdx.x * 256 + threadIdx.x;
  if (k >= nc) return;
  const float *aw = att + w * a_ws, *cw = cla + w * a_ws;
  float mx = -3.402823466e38f;
  for (int t = 0; t < Lt; t++) {
    float a2 = aw[(long long)t * ncp + k];
    a2 = a2 < -10.f ? -10.f : (a2 > 10.f ? 10.f : a2);
    mx = bnh_fmaxnm(mx, a2);
  }
  float z = 0.f, acc = 0.f;
  for (int t = 0; t < Lt; t++) {
    float a2 = aw[(long long)t * ncp + k];
    a2 = a2 < -10.f ? -10.f : (a2 > 10.f ? 10.f : a2);
    const float ev = bnh_expf(a2 - mx);
    z += ev;
    acc += ev * cw[(long long)t * ncp + k];
  }
  float *lw = logits + w * l_ws;
  lw[k] = lw[k] + acc / z;
}

// ------------------------------------------------------------------ SE gate with fp16-held weights (SE_GATE16)
// src/rt_ops_dot.c:381-420, one block per window: chsum scaled in place (x (1 / P)); fc1 per r: 8 fp32 FMA chains
// over 8-channel steps (lanes 0-3 and 4-7 of the reference's two accumulators), lane pairs added, then
// ((l0 + l1) + (l2 + l3)) + b1, SiLU v / (1 + expf(-v)); fc2 per channel from b2, one FMA per r in order; sigmoid by
// exp2_p5, FRECPE and two Newton steps; rounded to fp16.
__global__ __launch_bounds__(256) void k_se_gate16(float *__restrict__ chsum, long long c_ws, int C, int rd, float inv,
                                                   const uint16_t *__restrict__ w1, const float *__restrict__ b1,
                                                   const uint16_t *__restrict__ w2t, const float *__restrict__ b2,
                                                   uint16_t *__restrict__ gate, long long g_ws) {
  extern __shared__ float s_se[];  // [C] means, then [rd] fc1 outputs
  const int w = blockIdx.x;
  float *cs = chsum + w * c_ws;
  float *m = s_se, *tmp = s_se + C;
  for (int ch = threadIdx.x; ch < C; ch += 256) {
    const float v = cs[ch] * inv;
    m[ch] = v;
    cs[ch] = v;
  }
  __syncthreads();
  for (int r = threadIdx.x; r < rd; r += 256) {
    const uint16_t *wr = w1 + (long long)r * C;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int ch = 0; ch < C; ch += 8) {
#pragma unroll
      for (int l = 0; l < 8; l++) acc[l] = __builtin_fmaf((float)hfrom(wr[ch + l]), m[ch + l], acc[l]);
    }
    const float s0 = acc[0] + acc[4], s1 = acc[1] + acc[5], s2 = acc[2] + acc[6], s3 = acc[3] + acc[7];
    const float v = ((s0 + s1) + (s2 + s3)) + b1[r];
    tmp[r] = v / (1.f + bnh_expf(-v));
  }
  __syncthreads();
  for (int ch = threadIdx.x; ch < C; ch += 256) {
    float g = b2[ch];
    for (int r = 0; r < rd; r++) g = __builtin_fmaf((float)hfrom(w2t[(long long)r * C + ch]), tmp[r], g);
    gate[w * g_ws + ch] = hbits(f2h(qd_rcp1p_exp2(g * -1.44269504f)));
  }
}

// ------------------------------------------------------------------ generalised mean (GEM_A, src/rt_ops_dot.c:439-465)
// e[c] = powf(mean over rows of exp2_p5(max(p log2(max(F, eps)), -126)), 1 / p): the sums in row order from 0; the
// final power with the C library's powf results (bnh_powf.h: glibc's table method, restated)
__global__ __launch_bounds__(256) void k_gem_a(const float *__restrict__ F, long long f_ws, int M, int C, float eps,
                                               float p, float *__restrict__ e, long long e_ws) {
  const int w = blockIdx.y, ch = blockIdx.x * 256 + threadIdx.x;
  if (ch >= C) return;
  const float *Fw = F + w * f_ws;
  float acc = 0.f;
  for (int i = 0; i < M; i++) {
    const float v = bnh_fmax(Fw[(long long)i * C + ch], eps);
    acc = acc + qd_exp2_p5(bnh_fmax(p * qd_log2(v), -126.f));
  }
  const float mean = acc / (float)M, ip = 1.0f / p;
  e[w * e_ws + ch] = bnh_powf(mean, ip);
}

// ------------------------------------------------------------------ host side
extern "C" {

// qw_pack (src/gemm_s8.c:10-35) into [Np][Kp] rows; channels N..Np-1 are the zero rows of pack_padded
// (src/rt_ops_dot.c:467-473)
bnh_qdw *bnh_qdw_new(const float *w, const float *bias, int N, int K, int Np) {
  if (!w || N <= 0 || K <= 0 || K > (1 << 20) || Np < N || Np % 16) {
    bnh_fail("bnh_qdw_new: N %d K %d Np %d: expected N > 0, 0 < K <= 2^20, Np >= N, Np %% 16 == 0 and the weights",
             N, K, Np);
    return nullptr;
  }
  const int Kp = (K + 15) & ~15;
  int8_t *hq = (int8_t *)calloc((size_t)Np * Kp, 1);
  float *hs = (float *)calloc(Np, 4), *hss = (float *)calloc(Np, 4), *hb = (float *)calloc(Np, 4);
  bnh_qdw *W = (bnh_qdw *)calloc(1, sizeof *W);
  if (!hq || !hs || !hss || !hb || !W) {
    free(hq); free(hs); free(hss); free(hb); free(W);
    bnh_fail("bnh_qdw_new: out of host memory");
    return nullptr;
  }
  for (int n = 0; n < Np; n++) {
    float mx = 0.f;
    if (n < N)
      for (int k = 0; k < K; k++) mx = fmaxf(mx, fabsf(w[(size_t)n * K + k]));
    const float s = mx > 0.f ? mx / 127.f : 1.f;
    int32_t sum = 0;
    if (n < N)
      for (int k = 0; k < K; k++) {
        int v = (int)nearbyintf(w[(size_t)n * K + k] / s);
        v = v > 127 ? 127 : (v < -127 ? -127 : v);
        sum += v;
        hq[(size_t)n * Kp + k] = (int8_t)v;
      }
    hs[n] = s;
    hss[n] = s * (float)sum;
    hb[n] = bias && n < N ? bias[n] : 0.f;
  }
  W->N = N; W->K = K; W->Kp = Kp; W->Np = Np;
  bool ok = (W->w = (int8_t *)bnh_malloc((size_t)Np * Kp)) && (W->scale = (float *)bnh_malloc(4 * (size_t)Np)) &&
            (W->swsum = (float *)bnh_malloc(4 * (size_t)Np)) && (W->bias = (float *)bnh_malloc(4 * (size_t)Np)) &&
            !bnh_memcpy_h2d(W->w, hq, (size_t)Np * Kp) && !bnh_memcpy_h2d(W->scale, hs, 4 * (size_t)Np) &&
            !bnh_memcpy_h2d(W->swsum, hss, 4 * (size_t)Np) && !bnh_memcpy_h2d(W->bias, hb, 4 * (size_t)Np);
  free(hq); free(hs); free(hss); free(hb);
  if (!ok) { bnh_qdw_free(W); return nullptr; }
  return W;
}
void bnh_qdw_free(bnh_qdw *W) {
  if (!W) return;
  if (W->w) (void)hipFree(W->w);
  if (W->scale) (void)hipFree(W->scale);
  if (W->swsum) (void)hipFree(W->swsum);
  if (W->bias) (void)hipFree(W->bias);
  free(W);
}
int bnh_qdw_shape(const bnh_qdw *W, int *N, int *K, int *Kp, int *Np) {
  BNH_REQ(W);
  if (N) *N = W->N;
  if (K) *K = W->K;
  if (Kp) *Kp = W->Kp;
  if (Np) *Np = W->Np;
  return 0;
}

int bnh_qd_quant_rows(const void *x, int in_f16, long long x_ws, int ldx, int M, int K, const uint16_t *gate,
                      long long g_ws, int8_t *a, long long a_ws, float *rq, long long rq_ws, int B, void *stream) {
  BNH_REQ(x && a && rq && M > 0 && K > 0 && B > 0 && B <= 65535 && ldx >= K && (in_f16 == 0 || in_f16 == 1));
  BNH_REQ(!gate || in_f16);
  const int Kp = (K + 15) & ~15;
  BNH_REQ(((uintptr_t)a & 3) == 0 && (B == 1 || (a_ws % 4 == 0 && a_ws >= (long long)M * Kp)));
  BNH_REQ(B == 1 || (x_ws >= (long long)(M - 1) * ldx + K && rq_ws >= 2LL * M && (!gate || g_ws >= K)));
  const long long rows = (long long)M * B;
  // the vector form: 8-channel chunks (16-byte aligned rows of fp16, 32-byte of fp32; 8-byte aligned code rows)
  const int esz = in_f16 ? 2 : 4;
  const bool vec = K % 8 == 0 && ((uintptr_t)x & 15) == 0 && (ldx * esz) % 16 == 0 && (B == 1 || (x_ws * esz) % 16 == 0) &&
                   (!gate || (((uintptr_t)gate & 15) == 0 && (B == 1 || (g_ws * 2) % 16 == 0))) &&
                   ((uintptr_t)a & 7) == 0 && (B == 1 || a_ws % 8 == 0);
  if (vec) {
    int L = 1;
    while (L < 64 && 8 * L < K) L *= 2;  // lanes per row: enough for one pass over K where that fits in a wave
    const unsigned nbv = (unsigned)bnh_ceil_div(rows * L, 256);
    hipStream_t st = bnh_stream(stream);
#define QDQ(LL)                                                                                                        \
  if (L == LL) {                                                                                                      \
    if (in_f16)                                                                                                        \
      hipLaunchKernelGGL((k_qd_quant_v<LL, true>), dim3(nbv), dim3(256), 0, st, x, x_ws, ldx, M, 1.0 / M, K, Kp,       \
                         gate, g_ws, a, a_ws, rq, rq_ws, rows);                                                        \
    else                                                                                                               \
      hipLaunchKernelGGL((k_qd_quant_v<LL, false>), dim3(nbv), dim3(256), 0, st, x, x_ws, ldx, M, 1.0 / M, K, Kp,      \
                         nullptr, 0LL, a, a_ws, rq, rq_ws, rows);                                                      \
  }
    QDQ(1) QDQ(2) QDQ(4) QDQ(8) QDQ(16) QDQ(32) QDQ(64)
#undef QDQ
    BNH_HIP(hipGetLastError());
    return 0;
  }
  const unsigned nb = (unsigned)bnh_ceil_div(rows, 4);
  if (in_f16)
    hipLaunchKernelGGL(k_qd_quant<true>, dim3(nb), dim3(256), 0, bnh_stream(stream), x, x_ws, ldx, M, 1.0 / M, K, Kp,
                       gate, g_ws, a, a_ws, rq, rq_ws, rows);
  else
    hipLaunchKernelGGL(k_qd_quant<false>, dim3(nb), dim3(256), 0, bnh_stream(stream), x, x_ws, ldx, M, 1.0 / M, K,
                       Kp, nullptr, 0LL, a, a_ws, rq, rq_ws, rows);
  BNH_HIP(hipGetLastError());
  return 0;
}

static int qd_gemm_launch(bool conv, const int8_t *a, long long a_ws, int lda, const float *rq, long long rq_ws,
                          int per_tensor, int M, const bnh_qdw *W, const bnh_qd_epi *e, const QdConv &cv, int B,
                          void *stream) {
  BNH_REQ(a && rq && W && e && e->out && M > 0 && B > 0 && B <= 65535);
  BNH_REQ(e->act >= 0 && e->act <= 2 && (e->out_f16 == 0 || e->out_f16 == 1) && (!e->out_f16 || e->act != 2));
  BNH_REQ(e->ldo >= W->Np && e->opad >= 0 && e->opad <= 1 && (!e->opad || (e->ow > 0 && M % e->ow == 0)));
  BNH_REQ(!e->res || (!e->out_f16 && !e->opad));
  BNH_REQ(((uintptr_t)a & 15) == 0 && (conv || (lda % 16 == 0 && lda >= W->Kp)));
  BNH_REQ(B == 1 || (a_ws % 16 == 0 && rq_ws >= (per_tensor ? 2 : 2LL * M)));
  BNH_REQ(B == 1 || (e->out_ws >= (long long)(e->opad ? (M / e->ow + 2) * (e->ow + 2) : M) * e->ldo &&
                     (!e->res || e->res_ws >= (long long)M * e->ldo)));
  const long long rows = (long long)M * B;
  const int nrb = (int)bnh_ceil_div(rows, 128), ng = W->Np / 64 + (W->Np % 64 ? 1 : 0);
  int gsplit = 1;
  if (nrb < 1024) gsplit = (int)bnh_ceil_div(1024, nrb);
  if (gsplit > ng) gsplit = ng;
  BNH_REQ((long long)nrb * gsplit < (1LL << 31));
  QdEpi d = {e->act, e->out_f16, e->out, e->out_ws, e->ldo, e->ow, e->opad, e->ow > 0 ? 1.0 / e->ow : 0.0, e->res,
             e->res_ws};
  const dim3 grid((unsigned)(nrb * gsplit));
  // 16-byte row chunks: 16-byte aligned rows (8 halves / 4 floats) in the output and the residual
  const int esz = e->out_f16 ? 2 : 4;
  const bool vec = ((uintptr_t)e->out & 15) == 0 && (e->ldo * esz) % 16 == 0 && (B == 1 || (e->out_ws * esz) % 16 == 0) &&
                   (!e->res || (((uintptr_t)e->res & 15) == 0 && (B == 1 || e->res_ws % 4 == 0)));
#define QDG(CV, VC)                                                                                                    \
  hipLaunchKernelGGL((k_qd_gemm<CV, VC>), grid, dim3(256), 0, bnh_stream(stream), a, a_ws, lda, rq, rq_ws, per_tensor, \
                     M, 1.0 / M, rows, W->w, W->scale, W->swsum, W->bias, W->Kp, W->Np, gsplit, d, cv)
  if (conv) {
    if (vec) QDG(true, true);
    else QDG(true, false);
  } else {
    if (vec) QDG(false, true);
    else QDG(false, false);
  }
#undef QDG
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_qd_gemm(const int8_t *a, long long a_ws, int lda, const float *rq, long long rq_ws, int per_tensor, int M,
                const bnh_qdw *W, const bnh_qd_epi *e, int B, void *stream) {
  QdConv cv = {0, 1, 0, 0, 1, 1, 1.0};
  return qd_gemm_launch(false, a, a_ws, lda, rq, rq_ws, per_tensor ? 1 : 0, M, W, e, cv, B, stream);
}

size_t bnh_qconv3_work_bytes(int H, int W, int C) {
  return 1024 + (size_t)bnh_round_up((long long)(H + 2) * (W + 2) * C, 256);
}
int bnh_qconv3(const float *x, long long x_ws, int H, int W, int C, int s, int pt, int pl, int Ho, int Wo,
               const bnh_qdw *Wq, uint16_t *out, long long o_ws, int B, void *work, size_t work_ws, void *stream) {
  BNH_REQ(x && Wq && out && work && H > 0 && W > 0 && C > 0 && C % 8 == 0 && (s == 1 || s == 2) && B > 0 &&
          B <= 65535);
  BNH_REQ(Wq->K == 9 * C && Wq->N == Wq->Np && Ho > 0 && Wo > 0);
  BNH_REQ((Ho - 1) * s + 2 - pt <= H && (Wo - 1) * s + 2 - pl <= W && pt >= 0 && pt <= 1 && pl >= 0 && pl <= 1);
  BNH_REQ(work_ws >= bnh_qconv3_work_bytes(H, W, C) && work_ws % 256 == 0 && ((uintptr_t)work & 255) == 0);
  BNH_REQ(B == 1 || (x_ws >= (long long)H * W * C && o_ws >= (long long)Ho * Wo * Wq->Np));
  const long long n = (long long)H * W * C;
  const int nbk = (int)(n / 16384 < 1 ? 1 : (n / 16384 > 64 ? 64 : n / 16384));
  const long long nq = (long long)(H + 2) * (W + 2) * C / 4;
  const int nbq = (int)(nq / 4096 < 1 ? 1 : (nq / 4096 > 256 ? 256 : nq / 4096));
  char *wk = (char *)work;
  // per window slot of work_ws bytes: up to 64 partial (min, max) pairs, (scale, zp) at byte 768, the copy at 1024
  float *part = (float *)wk, *rq = (float *)(wk + 768);
  int8_t *xp = (int8_t *)(wk + 1024);
  const long long ws = (long long)work_ws;
  hipStream_t st = bnh_stream(stream);
  hipLaunchKernelGGL(k_qd_tminmax, dim3(nbk, B), dim3(256), 0, st, x, x_ws, n, nbk, part, ws / 4);
  BNH_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_qd_tquant, dim3(nbq, B), dim3(256), 0, st, x, x_ws, H, W, C, part, ws / 4, nbk, xp, ws, rq,
                     ws / 4, nbq);
  BNH_HIP(hipGetLastError());
  bnh_qd_epi e = {1, 1, out, o_ws, Wq->Np, 0, 0, nullptr, 0};
  const QdConv cv = {C, s, pt, pl, Wo, W + 2, 1.0 / Wo};
  return qd_gemm_launch(true, xp, ws, 0, rq, ws / 4, 1, Ho * Wo, Wq, &e, cv, B, stream);
}

// the SED heads: 7 weight sets (lin, then fc, att, cla of the head over H and of the head over W)
struct bnh_heads8 {
  int C, hid, nc, ncp;
  bnh_qdw *W[7];
};
bnh_heads8 *bnh_heads8_new(int C, int hid, int nc, const float *const *w, const float *const *b) {
  if (C <= 0 || C % 16 || hid <= 0 || hid % 16 || nc <= 0 || !w || !b) {
    bnh_fail("bnh_heads8_new: C %d hid %d nc %d: expected C %% 16 == 0, hid %% 16 == 0, nc > 0 and the tensors", C,
             hid, nc);
    return nullptr;
  }
  bnh_heads8 *P = (bnh_heads8 *)calloc(1, sizeof *P);
  if (!P) {
    bnh_fail("bnh_heads8_new: out of host memory");
    return nullptr;
  }
  P->C = C; P->hid = hid; P->nc = nc; P->ncp = (nc + 15) & ~15;
  for (int i = 0; i < 7; i++) {
    const int kind = i == 0 ? 0 : (i - 1) % 3;  // 0: [nc][C] (lin) / [hid][C] (fc), 1 / 2: [nc][hid]
    const int N = i == 0 ? nc : (kind == 0 ? hid : nc), K = kind == 0 ? C : hid, Np = i == 0 || kind ? P->ncp : hid;
    if (!(P->W[i] = bnh_qdw_new(w[i], b[i], N, K, Np))) {
      bnh_heads8_free(P);
      return nullptr;
    }
  }
  return P;
}
void bnh_heads8_free(bnh_heads8 *P) {
  if (!P) return;
  for (int i = 0; i < 7; i++) bnh_qdw_free(P->W[i]);
  free(P);
}
size_t bnh_heads8_work_bytes(int H, int W, int C, int hid, int nc) {
  const long long L = H > W ? H : W, ncp = (nc + 15) & ~15;
  return (size_t)bnh_round_up(4 * L * (2LL * C + hid + 2 * ncp), 256);
}
int bnh_heads_s8(const float *F, long long f_ws, const float *emb, long long e_ws, int H, int W, const bnh_heads8 *P,
                 float *logits, long long l_ws, int8_t *a8, long long a8_ws, float *rq, long long rq_ws, int B,
                 void *work, size_t work_ws, void *stream) {
  BNH_REQ(F && emb && P && logits && a8 && rq && work && H > 0 && W > 0 && B > 0 && B <= 65535);
  const int C = P->C, hid = P->hid, ncp = P->ncp, L = H > W ? H : W;
  const int kq = C > hid ? C : hid;
  BNH_REQ(work_ws >= bnh_heads8_work_bytes(H, W, C, hid, P->nc) && work_ws % 16 == 0);
  BNH_REQ(B == 1 || (f_ws >= (long long)H * W * C && e_ws >= C && l_ws >= ncp && a8_ws >= (long long)(L + 4) * kq &&
                     rq_ws >= 2LL * (L + 4)));
  const long long ws = (long long)work_ws / 4;  // floats per window slot
  float *wk = (float *)work;
  float *s = wk, *pooled = s + (long long)L * C, *h = pooled + (long long)L * C, *att = h + (long long)L * hid;
  float *cla = att + (long long)L * ncp;
  hipStream_t st = bnh_stream(stream);
  // lin(e) into the logits
  if (bnh_qd_quant_rows(emb, 0, e_ws, C, 1, C, nullptr, 0, a8, a8_ws, rq, rq_ws, B, stream)) return -1;
  bnh_qd_epi el = {0, 0, logits, l_ws, ncp, 0, 0, nullptr, 0};
  if (bnh_qd_gemm(a8, a8_ws, C, rq, rq_ws, 0, 1, P->W[0], &el, B, stream)) return -1;
  for (int i = 0; i < 2; i++) {
    const int Lt = i == 0 ? H : W;
    const dim3 g2((unsigned)bnh_ceil_div((long long)Lt * C, 256), (unsigned)B);
    if (i == 0) hipLaunchKernelGGL(k_hd_means<0>, g2, dim3(256), 0, st, F, f_ws, H, W, C, s, ws);
    else hipLaunchKernelGGL(k_hd_means<1>, g2, dim3(256), 0, st, F, f_ws, H, W, C, s, ws);
    BNH_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_hd_pool, g2, dim3(256), 0, st, s, ws, Lt, C, pooled, ws);
    BNH_HIP(hipGetLastError());
    if (bnh_qd_quant_rows(pooled, 0, ws, C, Lt, C, nullptr, 0, a8, a8_ws, rq, rq_ws, B, stream)) return -1;
    bnh_qd_epi ef = {2, 0, h, ws, hid, 0, 0, nullptr, 0};
    if (bnh_qd_gemm(a8, a8_ws, C, rq, rq_ws, 0, Lt, P->W[1 + 3 * i], &ef, B, stream)) return -1;
    if (bnh_qd_quant_rows(h, 0, ws, hid, Lt, hid, nullptr, 0, a8, a8_ws, rq, rq_ws, B, stream)) return -1;
    bnh_qd_epi ea = {0, 0, att, ws, ncp, 0, 0, nullptr, 0};
    if (bnh_qd_gemm(a8, a8_ws, hid, rq, rq_ws, 0, Lt, P->W[2 + 3 * i], &ea, B, stream)) return -1;
    bnh_qd_epi ec = {0, 0, cla, ws, ncp, 0, 0, nullptr, 0};
    if (bnh_qd_gemm(a8, a8_ws, hid, rq, rq_ws, 0, Lt, P->W[3 + 3 * i], &ec, B, stream)) return -1;
    hipLaunchKernelGGL(k_hd_softmax, dim3((unsigned)bnh_ceil_div(P->nc, 256), (unsigned)B), dim3(256), 0, st, att,
                       cla, ws, Lt, ncp, P->nc, logits, l_ws);
    BNH_HIP(hipGetLastError());
  }
  return 0;
}

// the SE gate's weights held in fp16 (rounded to nearest even), fc2 transposed to [rd][C]
struct bnh_seg16 {
  int C, rd;
  uint16_t *w1, *w2t;
  float *b1, *b2;
};
bnh_seg16 *bnh_seg16_new(int C, int rd, const float *w1, const float *b1, const float *w2, const float *b2) {
  if (C <= 0 || C % 8 || rd <= 0 || C + rd > 16384 || !w1 || !b1 || !w2 || !b2) {
    bnh_fail("bnh_seg16_new: C %d rd %d: expected C %% 8 == 0, rd > 0, C + rd <= 16384 and all four tensors", C, rd);
    return nullptr;
  }
  const size_t n = (size_t)C * rd;
  uint16_t *h1 = (uint16_t *)malloc(2 * n), *h2 = (uint16_t *)malloc(2 * n);
  bnh_seg16 *S = (bnh_seg16 *)calloc(1, sizeof *S);
  if (!h1 || !h2 || !S) {
    free(h1); free(h2); free(S);
    bnh_fail("bnh_seg16_new: out of host memory");
    return nullptr;
  }
  for (int r = 0; r < rd; r++)
    for (int ch = 0; ch < C; ch++) {
      const _Float16 a = (_Float16)w1[(size_t)r * C + ch], b = (_Float16)w2[(size_t)ch * rd + r];
      memcpy(&h1[(size_t)r * C + ch], &a, 2);
      memcpy(&h2[(size_t)r * C + ch], &b, 2);
    }
  S->C = C; S->rd = rd;
  bool ok = (S->w1 = (uint16_t *)bnh_malloc(2 * n)) && (S->w2t = (uint16_t *)bnh_malloc(2 * n)) &&
            (S->b1 = (float *)bnh_malloc(4 * (size_t)rd)) && (S->b2 = (float *)bnh_malloc(4 * (size_t)C)) &&
            !bnh_memcpy_h2d(S->w1, h1, 2 * n) && !bnh_memcpy_h2d(S->w2t, h2, 2 * n) &&
            !bnh_memcpy_h2d(S->b1, b1, 4 * (size_t)rd) && !bnh_memcpy_h2d(S->b2, b2, 4 * (size_t)C);
  free(h1); free(h2);
  if (!ok) { bnh_seg16_free(S); return nullptr; }
  return S;
}
void bnh_seg16_free(bnh_seg16 *S) {
  if (!S) return;
  if (S->w1) (void)hipFree(S->w1);
  if (S->w2t) (void)hipFree(S->w2t);
  if (S->b1) (void)hipFree(S->b1);
  if (S->b2) (void)hipFree(S->b2);
  free(S);
}
int bnh_se_gate16(float *chsum, long long c_ws, int P, const bnh_seg16 *S, uint16_t *gate, long long g_ws, int B,
                  void *stream) {
  BNH_REQ(chsum && S && gate && P > 0 && B > 0 && B <= 65535);
  BNH_REQ(B == 1 || (c_ws >= S->C && g_ws >= S->C));
  const float inv = 1.f / (float)P;
  hipLaunchKernelGGL(k_se_gate16, dim3(B), dim3(256), (size_t)(S->C + S->rd) * 4, bnh_stream(stream), chsum, c_ws,
                     S->C, S->rd, inv, S->w1, S->b1, S->w2t, S->b2, gate, g_ws);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_gem_a(const float *F, long long f_ws, int M, int C, float eps, float p, float *e, long long e_ws, int B,
              void *stream) {
  BNH_REQ(F && e && M > 0 && C > 0 && B > 0 && B <= 65535);
  BNH_REQ(B == 1 || (f_ws >= (long long)M * C && e_ws >= C));
  hipLaunchKernelGGL(k_gem_a, dim3((unsigned)bnh_ceil_div(C, 256), (unsigned)B), dim3(256), 0, bnh_stream(stream), F,
                     f_ws, M, C, eps, p, e, e_ws);
  BNH_HIP(hipGetLastError());
  return 0;
}

// device forms of the scalar functions, elementwise (their parity tests): 0 exp2_p5, 1 silu_f32_a, 2 log2, 3 the
// SE gate's sigmoid of x
__global__ void k_eval_qd(int f, const float *__restrict__ x, float *__restrict__ y, long long n) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  y[i] = f == 0 ? qd_exp2_p5(v) : f == 1 ? qd_silu_f32_a(v) : f == 2 ? qd_log2(v) : qd_rcp1p_exp2(v * -1.44269504f);
}
int bnh_eval_qd(int f, const float *x, float *y, long long n, void *stream) {
  BNH_REQ(x && y && n > 0 && f >= 0 && f <= 3);
  hipLaunchKernelGGL(k_eval_qd, dim3((unsigned)bnh_ceil_div(n, 256)), dim3(256), 0, bnh_stream(stream), f, x, y, n);
  BNH_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
