// int8 pointwise-convolution GEMMs on gfx950 int8 MFMA (v_mfma_i32_16x16x64_i8, exact int32 accumulation).
//
//  * PW_S8 (libbnneon's int8 GEMM without dotprod, src/gemm_s8n.c + src/rt_ops_s8n.c): fp32 NHWC rows quantized
//    per row (dynamic, asymmetric into [-127, 127]), per-channel symmetric int8 weights, fp32 dequant epilogue with
//    SiLU / ReLU / residual / zero-haloed store. Bit-identical to the reference for every input.
//  * the Q31-requantised static int8 GEMM (NCHW, int8 out): this library's own specification (bnneon_hip.h).
//
// Layouts in HBM:
//  * q rows [M][Kp] per window (K contiguous) are the MFMA A operand as they stand: lane l of a 16x16x64 MFMA
//    takes 16 bytes of row (l & 15) at k offset 16 (l >> 4) -- the same k chunk rule for A and B, so the int32 sums
//    are exact whatever order the matrix core adds them in.
//  * weights are repacked at load from the package's [Np/4][Kp/16][4][16] panels into channel rows [Nt][Kp]
//    (Nt = Np rounded up to 128, zero rows beyond Np): lane l loads channel (l & 15), the same 16-byte k chunk.
//  * per-channel epilogue vectors (sw, colsum, b) padded to Nt with zeros.
// Tiles: a wave computes 32 rows x 64 channels (2 x 4 MFMA tiles, 32 accumulator registers); 4 waves per block.
#include <string.h>

#include "bnh_internal.h"
#include "bnh_num.h"
#include "bnh_lds_dma.h"

typedef int v4i __attribute__((ext_vector_type(4)));

struct bnh_q8w {
  int N, K, Kt, Nt, zx, zy, lo, hi;
  int all_s1;         // every shift in 1..31: the epilogues need only the one-rounding form
  int8_t *w;          // [Nt][Kt], zero past K (Kt = K rounded up to 64) and past N
  int32_t *bias_eff;  // [Nt]: bias[n] - zx * sum_k w[n][k] (wrapping int32)
  int32_t *mult, *shift;
  // the short epilogue (every shift in 1..31, zy <= lo, and |bias_eff| + K 2^14 < 2^31 so that acc + bias_eff never
  // wraps): cq[n] = bias_eff[n] mult[n] + 2^30 + 2^(30 + shift[n]) and e1[n] = shift[n] - 1, so a requantised output
  // is zy + clamp((acc mult + cq) >> (32 + e1), lo - zy, hi - zy)
  int fast;
  int32_t *cq;  // [2 Nt]: the low words of cq, then the high words
  int32_t *e1;
};

struct EpiDev {  // the fp32 epilogue, by value into the kernel
  int act;
  float *out;
  long long out_ws;
  int ldo, ow, opad;
  const float *res;
  long long res_ws;
  int ldr, rpad, rw;
  double r_ow, r_rw;  // 1 / ow, 1 / rw (padded row arithmetic)
  int vec;            // k_s8n_gemm: rows stored (and residuals read) as 16-byte quads through LDS
};

// the padded row of pixel m (ow pixels per image row, halo opad)
BNH_DEV long long epi_prow(int m, int ow, int opad, double r_ow) {
  if (!opad) return m;
  const int y = bnh_div(m, ow, r_ow);
  return (long long)(y + opad) * (ow + 2 * opad) + (m - y * ow) + opad;
}

// ------------------------------------------------------------------ per-row quantization (s8n_quant_rows)
// One wavefront per row. min / max over k < K & ~3 with FMIN / FMAX semantics (any order: both are exact and, for
// the values they can return, associative), then the K % 4 tail in order with FMINNM / FMAXNM, as the reference's
// 4-lane loop + scalar tail. Quantization: FCVTNS for k < K & ~7, (int32_t)lrintf for the K % 8 tail.
__global__ __launch_bounds__(256) void k_s8n_quant(const float *__restrict__ x, long long x_ws, int ld, int M, int K,
                                                   int Kp, const float *__restrict__ gate, long long g_ws,
                                                   int8_t *__restrict__ q, long long q_ws, float *__restrict__ sa,
                                                   long long sa_ws, int32_t *__restrict__ za, long long za_ws,
                                                   long long rows) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int w = (int)(row / M), m = (int)(row % M);
  const float *r = x + w * x_ws + (long long)m * ld;
  const float *g = gate ? gate + w * g_ws : nullptr;
  const int K4 = K & ~3, K8 = K & ~7;
  float lo = __builtin_inff(), hi = -__builtin_inff();
  for (int k = lane; k < K4; k += 64) {
    float v = r[k];
    if (g) v = v * g[k];
    lo = bnh_fmin(lo, v);
    hi = bnh_fmax(hi, v);
  }
  for (int off = 32; off; off >>= 1) {
    lo = bnh_fmin(lo, __shfl_xor(lo, off));
    hi = bnh_fmax(hi, __shfl_xor(hi, off));
  }
  for (int k = K4; k < K; k++) {
    float v = r[k];
    if (g) v = v * g[k];
    lo = bnh_fminnm(lo, v);
    hi = bnh_fmaxnm(hi, v);
  }
  float inv, s;
  int32_t z;
  const float range = hi - lo;
  if (!(range > 1e-30f * bnh_fmaxnm(__builtin_fabsf(hi), __builtin_fabsf(lo))) || !(range > 0.f)) {
    float a = bnh_fmaxnm(__builtin_fabsf(hi), 1e-30f);
    inv = 127.f / a;
    z = 0;
    s = a / 127.f;
  } else {
    inv = 254.f / range;
    z = (int32_t)((uint32_t)-127 - (uint32_t)bnh_lrintf_s32(lo * inv));
    s = range / 254.f;
  }
  if (lane == 0) {
    sa[w * sa_ws + m] = s;
    za[w * za_ws + m] = z;
  }
  int8_t *o = q + w * q_ws + (long long)m * Kp;
  const uint32_t zb = (uint32_t)z & 0xffu;
  for (int k0 = lane * 4; k0 < Kp; k0 += 256) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int k = k0 + j;
      uint32_t byte;
      if (k < K) {
        float v = r[k];
        if (g) v = v * g[k];
        const float t = v * inv;
        int32_t c = (int32_t)((uint32_t)(k < K8 ? bnh_cvtn_s32(t) : bnh_lrintf_s32(t)) + (uint32_t)z);
        c = c < -127 ? -127 : c > 127 ? 127 : c;
        byte = (uint32_t)c & 0xffu;
      } else
        byte = zb;
      word |= byte << (8 * j);
    }
    *(uint32_t *)(o + k0) = word;
  }
}

// The same quantization with L lanes per row (L a power of two, 256 / L rows per block) and 16-byte loads, for rows
// whose start is 16-byte aligned: each lane takes every L-th 4-element chunk, min / max meet in an L-lane butterfly.
template <int L>
__global__ __launch_bounds__(256) void k_s8n_quant_v(const float *__restrict__ x, long long x_ws, int ld, int M, int K,
                                                     int Kp, const float *__restrict__ gate, long long g_ws,
                                                     int8_t *__restrict__ q, long long q_ws, float *__restrict__ sa,
                                                     long long sa_ws, int32_t *__restrict__ za, long long za_ws,
                                                     long long rows, double rM) {
  const int sub = threadIdx.x % L;
  const long long row0 = (long long)blockIdx.x * (256 / L) + threadIdx.x / L;
  const bool valid = row0 < rows;
  const long long row = valid ? row0 : rows - 1;  // every lane takes part in the butterfly
  const int w = bnh_div(row, M, rM), m = (int)(row - (long long)w * M);
  const float *r = x + w * x_ws + (long long)m * ld;
  const float *g = gate ? gate + w * g_ws : nullptr;
  const int K4 = K & ~3, K8 = K & ~7, n4 = K4 / 4;
  // min / max of k < K4: the reference's FMIN / FMAX give NaN when any element is NaN and otherwise the exact
  // extremes (the sign of a zero extreme changes no later result); fminf / fmaxf plus a NaN flag give the same
  float lo = __builtin_inff(), hi = -__builtin_inff();
  int nan = 0;
  // the lane's first QC chunks (all of them when L < 64: 16 L >= Kp) stay in registers for the quantization pass,
  // the gate already applied; chunks past them (L = 64, Kp > 1024) are read again there
  constexpr int QC = 4;
  float4 cv[QC];
  auto chunk = [&](int c) {
    float4 v = *(const float4 *)(r + 4 * c);
    if (g) {
      const float4 gv = *(const float4 *)(g + 4 * c);
      v.x = v.x * gv.x; v.y = v.y * gv.y; v.z = v.z * gv.z; v.w = v.w * gv.w;
    }
    return v;
  };
  auto minmax = [&](const float4 &v) {
    nan |= (v.x != v.x) | (v.y != v.y) | (v.z != v.z) | (v.w != v.w);
    lo = __builtin_fminf(__builtin_fminf(lo, v.x), __builtin_fminf(v.y, __builtin_fminf(v.z, v.w)));
    hi = __builtin_fmaxf(__builtin_fmaxf(hi, v.x), __builtin_fmaxf(v.y, __builtin_fmaxf(v.z, v.w)));
  };
#pragma unroll
  for (int j = 0; j < QC; j++) {
    const int c = sub + j * L;
    if (c < n4) cv[j] = chunk(c);  // every load first, then the reductions
  }
#pragma unroll
  for (int j = 0; j < QC; j++)
    if (sub + j * L < n4) minmax(cv[j]);
  for (int c = sub + QC * L; c < n4; c += L) minmax(chunk(c));
#pragma unroll
  for (int off = L / 2; off; off >>= 1) {
    lo = __builtin_fminf(lo, __shfl_xor(lo, off));
    hi = __builtin_fmaxf(hi, __shfl_xor(hi, off));
    nan |= __shfl_xor(nan, off);
  }
  if (nan) lo = hi = __builtin_nanf("");
  for (int k = K4; k < K; k++) {
    float v = r[k];
    if (g) v = v * g[k];
    nan |= v != v;
    lo = bnh_fminnm(lo, v);
    hi = bnh_fmaxnm(hi, v);
  }
  float inv, sc;
  int32_t z;
  const float range = hi - lo;
  if (!(range > 1e-30f * bnh_fmaxnm(__builtin_fabsf(hi), __builtin_fabsf(lo))) || !(range > 0.f)) {
    const float a = bnh_fmaxnm(__builtin_fabsf(hi), 1e-30f);
    inv = 127.f / a;
    z = 0;
    sc = a / 127.f;
  } else {
    inv = 254.f / range;
    z = (int32_t)((uint32_t)-127 - (uint32_t)bnh_lrintf_s32(lo * inv));
    sc = range / 254.f;
  }
  if (!valid) return;
  if (sub == 0) {
    sa[w * sa_ws + m] = sc;
    za[w * za_ws + m] = z;
  }
  // a row of finite values whose scaled extremes stay below 2^30 needs no saturation: the roundings are plain
  const bool fast = !nan && __builtin_fmaxf(__builtin_fabsf(lo), __builtin_fabsf(hi)) * inv < 1073741824.f;
  int8_t *o = q + w * q_ws + (long long)m * Kp;
  const uint32_t zb = (uint32_t)z & 0xffu;
#pragma unroll
  for (int j = 0; j < QC + 1; j++) {  // j < QC: chunk sub + j L from registers; j = QC: the chunks past them
   for (int c = sub + j * L; c < Kp / 4; c += L) {
    const int k0 = 4 * c;
    float v[4];
    if (k0 + 4 <= K4) {
      const float4 t = j < QC ? cv[j] : chunk(c);
      v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    } else {
#pragma unroll
      for (int jj = 0; jj < 4; jj++) {
        const int k = k0 + jj;
        v[jj] = 0.f;
        if (k < K) {
          v[jj] = r[k];
          if (g) v[jj] = v[jj] * g[k];
        }
      }
    }
    uint32_t word = 0;
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
      const int k = k0 + jj;
      uint32_t byte = zb;
      if (k < K) {
        const float t = v[jj] * inv;
        int32_t cq;
        if (fast) cq = (int32_t)__builtin_rintf(t) + z;
        else cq = (int32_t)((uint32_t)(k < K8 ? bnh_cvtn_s32(t) : bnh_lrintf_s32(t)) + (uint32_t)z);
        cq = cq < -127 ? -127 : cq > 127 ? 127 : cq;
        byte = (uint32_t)cq & 0xffu;
      }
      word |= byte << (8 * jj);
    }
    *(uint32_t *)(o + k0) = word;
    if (j < QC) break;  // one chunk per register slot
   }
  }
}

// ------------------------------------------------------------------ int8 GEMM + fp32 dequant epilogue
// A block owns 128 rows (pixels of consecutive windows); its threads first resolve each row's window, pixel,
// quantisation parameters and output / residual addresses into LDS (once per row). Each wave then owns 32 of the
// rows and walks the 64-channel groups [g0, g1) of its block: per group 2 x 4 i8 MFMA tiles over K and the
// reference's epilogue. A wave writing every channel of its rows, one group after the other, hands whole output rows
// to its L2, where their cache lines complete before they are written back (rows split between blocks leave partial
// lines, which cost HBM write rate). Blocks split the channel groups only when there are too few rows to fill the
// chip (gsplit blocks per row block, consecutive after the XCD remap so that they share an L2). Four waves per SIMD
// at least (112 VGPRs, no spill, where the compiler's own choice took 151 and three): the K loop waits on its
// fragment loads, and more waves hide that (the Perch-shaped net 11.68 -> 11.60 ms per 256 windows).
template <bool RES>
__global__ __launch_bounds__(256, 4) void k_s8n_gemm(const int8_t *__restrict__ q, long long q_ws,
                                                  const float *__restrict__ sa, long long sa_ws,
                                                  const int32_t *__restrict__ za, long long za_ws, int M, double rM,
                                                  long long rows, const int8_t *__restrict__ wt,
                                                  const float *__restrict__ sw, const int32_t *__restrict__ cs,
                                                  const float *__restrict__ bias, int Kp, int Np, int gsplit,
                                                  EpiDev e) {
  constexpr int RB = 128;
  __shared__ long long s_q[RB], s_o[RB], s_r[RB];
  __shared__ float s_sa[RB];
  __shared__ uint32_t s_z[RB], s_tbl[256];
  constexpr int TS = 68;  // the vector epilogue's tile row stride in floats (64 channels + 4)
  __shared__ float s_t[RES ? 4 : 1][RES ? 16 * TS : 1];  // (the form without residual stores values directly)
  bnh_silu_table(s_tbl);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const unsigned lb = gsplit > 1 ? bnh_xcd_block(blockIdx.x, gridDim.x) : blockIdx.x;
  const long long rowB = (long long)(lb / gsplit) * RB;
  const int ng = (Np + 63) / 64, part = (int)(lb % gsplit);
  const int g0 = part * ng / gsplit, g1 = (part + 1) * ng / gsplit;
  for (int i = threadIdx.x; i < RB; i += 256) {
    const long long row = rowB + i < rows ? rowB + i : rows - 1;  // rows past the end repeat the last row
    const int w = bnh_div(row, M, rM), m = (int)(row - (long long)w * M);
    s_q[i] = w * q_ws + (long long)m * Kp;
    s_o[i] = w * e.out_ws + epi_prow(m, e.ow, e.opad, e.r_ow) * e.ldo;
    s_r[i] = e.res ? w * e.res_ws + epi_prow(m, e.rw, e.rpad, e.r_rw) * e.ldr : 0;
    s_sa[i] = sa[w * sa_ws + m];
    s_z[i] = (uint32_t)za[w * za_ws + m];
  }
  __syncthreads();
  const int lr0 = wave * 32;  // the wave's first row within the block
  if (rowB + lr0 >= rows) return;
  const int kc = (lane >> 4) * 16;  // this lane's k chunk within a 64-wide step
  const int8_t *ap[2];
#pragma unroll
  for (int t = 0; t < 2; t++) ap[t] = q + s_q[lr0 + 16 * t + (lane & 15)] + kc;
  const int kmain = Kp & ~63;
  const bool kin = kmain + kc < Kp;  // this lane's chunk of the last partial step holds k < Kp
  // one K step (Kp <= 64, the expansions): the A fragments once for every group
  v4i a1[2];
  if (Kp <= 64) {
#pragma unroll
    for (int t = 0; t < 2; t++) a1[t] = kin ? *(const v4i *)(ap[t]) : (v4i){0, 0, 0, 0};
  }
  for (int g = g0; g < g1; g++) {
    const int n0 = 64 * g;
    const int jn = Np - n0 >= 64 ? 4 : (Np - n0 + 15) / 16;  // the 16-channel groups that hold channels < Np
    const int8_t *bp = wt + (long long)(n0 + (lane & 15)) * Kp + kc;
    v4i acc[2][4];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[t][j] = (v4i){0, 0, 0, 0};
    if (Kp <= 64) {
      v4i b[4];
#pragma unroll
      for (int j = 0; j < 4; j++) b[j] = kin && j < jn ? *(const v4i *)(bp + (long long)16 * j * Kp) : (v4i){0, 0, 0, 0};
#pragma unroll
      for (int t = 0; t < 2; t++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          if (j < jn) acc[t][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[t], b[j], acc[t][j], 0, 0, 0);
    } else {
      for (int k = 0; k < kmain; k += 64) {
        v4i a[2], b[4];
#pragma unroll
        for (int t = 0; t < 2; t++) a[t] = *(const v4i *)(ap[t] + k);
#pragma unroll
        for (int j = 0; j < 4; j++) b[j] = j < jn ? *(const v4i *)(bp + (long long)16 * j * Kp + k) : (v4i){0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int j = 0; j < 4; j++)
            if (j < jn) acc[t][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[j], acc[t][j], 0, 0, 0);
      }
      if (kmain < Kp) {  // the last partial step: chunks at or past Kp contribute zeros
        v4i a[2], b[4];
#pragma unroll
        for (int t = 0; t < 2; t++) a[t] = kin ? *(const v4i *)(ap[t] + kmain) : (v4i){0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; j++)
          b[j] = kin && j < jn ? *(const v4i *)(bp + (long long)16 * j * Kp + kmain) : (v4i){0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int j = 0; j < 4; j++)
            if (j < jn) acc[t][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[j], acc[t][j], 0, 0, 0);
      }
    }
    // epilogue (deq4 + activation + store_rows, src/gemm_s8n.c:105-135): acc[t][j][r] is row 16t + 4 (lane >> 4) + r,
    // channel n0 + 16j + (lane & 15)
    float swn[4], bn[4];
    int32_t csn[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + 16 * j + (lane & 15);
      swn[j] = sw[n];
      bn[j] = bias[n];
      csn[j] = cs[n];
    }
    if (RES && e.vec) {
      // the tile's 16 rows x 64 channels go through the wave's LDS tile: each value dequantised and activated in the
      // accumulator layout (the same operations as below), then read back as 16-byte quads of a row, its residual
      // quad added, and stored whole (4 times fewer memory instructions than one 4-byte access per value)
      float *T = s_t[wave];
      const int nq = ((Np - n0 < 64 ? Np - n0 : 64) + 3) / 4;  // quads holding channels < Np (Np % 4 == 0)
#pragma unroll
      for (int t = 0; t < 2; t++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int lr = lr0 + 16 * t + 4 * (lane >> 4) + r;
          const float s_a = s_sa[lr];
          const uint32_t z = s_z[lr];
#pragma unroll
          for (int j = 0; j < 4; j++) {
            if (j >= jn) break;
            const int32_t c = (int32_t)((uint32_t)acc[t][j][r] - (uint32_t)csn[j] * z);
            const float f = (float)c;
            const float scl = swn[j] * s_a;
            float y = f * scl;
            y = y + bn[j];
            if (e.act == 1) y = bnh_silu_f32_t(y, s_tbl);
            else if (e.act == 2) y = bnh_relu_f32(y);
            T[(4 * (lane >> 4) + r) * TS + 16 * j + (lane & 15)] = y;
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int qd = lane & 15;
        float4 rq[4];
        if (RES) {  // every residual quad of the tile first (out and res may alias: loads before any store)
#pragma unroll
          for (int it = 0; it < 4; it++) {
            const int lr = lr0 + 16 * t + 4 * it + (lane >> 4);
            rq[it] = qd < nq && rowB + lr < rows ? *(const float4 *)(e.res + s_r[lr] + n0 + 4 * qd)
                                                 : make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
#pragma unroll
        for (int it = 0; it < 4; it++) {
          const int rr = 4 * it + (lane >> 4), lr = lr0 + 16 * t + rr;
          if (qd < nq && rowB + lr < rows) {
            float4 y = *(const float4 *)(T + rr * TS + 4 * qd);
            if (RES) {
              y.x = y.x + rq[it].x;
              y.y = y.y + rq[it].y;
              y.z = y.z + rq[it].z;
              y.w = y.w + rq[it].w;
            }
            *(float4 *)(e.out + s_o[lr] + n0 + 4 * qd) = y;
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
      // RES: the residuals of the tile's 16 rows first: loads issued together, and before any store (which the compiler
      // may not move them past: out and res could alias), so their latency is paid once per tile, not per row
      float rv[4][4];
      if (RES) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int lr = lr0 + 16 * t + 4 * (lane >> 4) + r;
          const float *rrow = e.res + s_r[lr];
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int n = n0 + 16 * j + (lane & 15);
            rv[r][j] = j < jn && n < Np && rowB + lr < rows ? rrow[n] : 0.f;
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int lr = lr0 + 16 * t + 4 * (lane >> 4) + r;
        if (rowB + lr >= rows) continue;
        const float s_a = s_sa[lr];
        const uint32_t z = s_z[lr];
        float *orow = e.out + s_o[lr];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          if (j >= jn) break;
          const int n = n0 + 16 * j + (lane & 15);
          if (n >= Np) continue;
          const int32_t c = (int32_t)((uint32_t)acc[t][j][r] - (uint32_t)csn[j] * z);
          const float f = (float)c;
          const float scl = swn[j] * s_a;
          float y = f * scl;
          y = y + bn[j];
          if (e.act == 1) y = bnh_silu_f32_t(y, s_tbl);
          else if (e.act == 2) y = bnh_relu_f32(y);
          if (RES) y = y + rv[r][j];
          orow[n] = y;
        }
      }
    }
  }
}

// ------------------------------------------------------------------ int8 GEMM + fp32 dequant epilogue, large K
// For Kp > 64 the per-group K loop of k_s8n_gemm re-reads a row's int8 bytes once per 64-channel group and waits on
// every fragment load; here a block owns a tile of TR = 64 WM rows x TN = 128 WN channels (WM x WN = 4 waves, each
// 64 rows x 128 channels = 4 x 8 MFMA tiles, 128 accumulator registers) and walks K once: each 64-byte K step of the
// tile's rows and weight rows is fetched from global memory into registers while the previous step's MFMAs run, then
// staged in one of two LDS buffers (rows at an 80-byte stride: the 16 rows a fragment read serves land on disjoint
// bank groups). Chunks at or past Kp load as zeros. The epilogue is k_s8n_gemm's, element for element.
#define SL_STRIDE 80
template <int WM, int WN, bool RES>
__global__ __launch_bounds__(256, 2) void k_s8n_gemm_lds(const int8_t *__restrict__ q, long long q_ws,
                                                         const float *__restrict__ sa, long long sa_ws,
                                                         const int32_t *__restrict__ za, long long za_ws, int M,
                                                         double rM, long long rows, const int8_t *__restrict__ wt,
                                                         const float *__restrict__ sw, const int32_t *__restrict__ cs,
                                                         const float *__restrict__ bias, int Kp, int Np, int Nt, int nct,
                                                         EpiDev e) {
  constexpr int TR = 64 * WM, TN = 128 * WN;
  constexpr int ACH = TR * 4 / 256, BCH = TN * 4 / 256;  // 16-byte chunks per thread per K step
  __shared__ __attribute__((aligned(16))) int8_t lds[2][(TR + TN) * SL_STRIDE];
  __shared__ long long s_q[TR], s_o[TR], s_r[RES ? TR : 1];
  __shared__ float s_sa[TR];
  __shared__ uint32_t s_z[TR], s_tbl[256];
  bnh_silu_table(s_tbl);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  // logical block: the channel tiles of a row tile consecutive, and consecutive blocks on one XCD (they share the
  // tile's rows in L2)
  const unsigned lb = bnh_xcd_block(blockIdx.x, gridDim.x);
  const long long rowB = (long long)(lb / nct) * TR;
  const int n0 = (int)(lb % nct) * TN;
  for (int i = tid; i < TR; i += 256) {
    const long long row = rowB + i < rows ? rowB + i : rows - 1;  // rows past the end repeat the last row
    const int w = bnh_div(row, M, rM), m = (int)(row - (long long)w * M);
    s_q[i] = w * q_ws + (long long)m * Kp;
    s_o[i] = w * e.out_ws + epi_prow(m, e.ow, e.opad, e.r_ow) * e.ldo;
    if (RES) s_r[i] = w * e.res_ws + epi_prow(m, e.rw, e.rpad, e.r_rw) * e.ldr;
    s_sa[i] = sa[w * sa_ws + m];
    s_z[i] = (uint32_t)za[w * za_ws + m];
  }
  __syncthreads();
  // staging roles: chunk i = tid + 256 c of the step: row i / 4, 16-byte chunk i % 4
  v4i ra[ACH], rb[BCH];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int c = 0; c < ACH; c++) {
      const int i = tid + 256 * c, r = i >> 2, k = k0 + 16 * (i & 3);
      ra[c] = k < Kp ? *(const v4i *)(q + s_q[r] + k) : (v4i){0, 0, 0, 0};
    }
#pragma unroll
    for (int c = 0; c < BCH; c++) {
      const int i = tid + 256 * c, n = n0 + (i >> 2), k = k0 + 16 * (i & 3);
      rb[c] = k < Kp && n < Nt ? *(const v4i *)(wt + (long long)n * Kp + k) : (v4i){0, 0, 0, 0};
    }
  };
  auto stage = [&](int8_t *buf) {
#pragma unroll
    for (int c = 0; c < ACH; c++) {
      const int i = tid + 256 * c;
      *(v4i *)(buf + (i >> 2) * SL_STRIDE + 16 * (i & 3)) = ra[c];
    }
#pragma unroll
    for (int c = 0; c < BCH; c++) {
      const int i = tid + 256 * c;
      *(v4i *)(buf + (TR + (i >> 2)) * SL_STRIDE + 16 * (i & 3)) = rb[c];
    }
  };
  v4i acc[4][8];
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int j = 0; j < 8; j++) acc[t][j] = (v4i){0, 0, 0, 0};
  const int kc = (lane >> 4) * 16;
  fetch(0);
  stage(lds[0]);
  __syncthreads();
  int cur = 0;
  for (int k0 = 0; k0 < Kp; k0 += 64) {
    const bool more = k0 + 64 < Kp;
    if (more) fetch(k0 + 64);  // in flight during this step's MFMAs
    const int8_t *as = lds[cur], *bs = lds[cur] + TR * SL_STRIDE;
    v4i a[4];
#pragma unroll
    for (int t = 0; t < 4; t++) a[t] = *(const v4i *)(as + (wm * 64 + 16 * t + (lane & 15)) * SL_STRIDE + kc);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const v4i b = *(const v4i *)(bs + (wn * 128 + 16 * j + (lane & 15)) * SL_STRIDE + kc);
#pragma unroll
      for (int t = 0; t < 4; t++) acc[t][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b, acc[t][j], 0, 0, 0);
    }
    if (more) {
      stage(lds[cur ^ 1]);  // the other buffer: its last reads were before the previous barrier
      __syncthreads();
      cur ^= 1;
    }
  }
  // epilogue (deq4 + activation + store_rows, src/gemm_s8n.c:105-135): acc[t][j][r] is row wm 64 + 16 t + 4 (lane >>
  // 4) + r, channel n0 + wn 128 + 16 j + (lane & 15)
  float swn[8], bn[8];
  int32_t csn[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int n = n0 + wn * 128 + 16 * j + (lane & 15);
    const bool in = n < Np;
    swn[j] = in ? sw[n] : 0.f;
    bn[j] = in ? bias[n] : 0.f;
    csn[j] = in ? cs[n] : 0;
  }
  if (e.vec) {
    // each 16-row tile through the wave's part of the (now idle) LDS buffers, [16][132] floats: the values
    // dequantised and activated in the accumulator layout, then read back as 16-byte quads of a row (residual quads
    // added) and stored whole, so every instruction writes whole 256-byte runs of rows
    constexpr int TS = 132;
    __syncthreads();  // every wave's last MFMA operand reads are done
    float *T = (float *)&lds[0][0] + wave * 16 * TS;
    const int nlim = Np - (n0 + wn * 128);  // channels of this wave's 128 that exist (a multiple of 4)
    const int nq = (nlim < 128 ? nlim : 128) / 4;
#pragma unroll
    for (int t = 0; t < 4; t++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int lr = wm * 64 + 16 * t + 4 * (lane >> 4) + r;
        const float s_a = s_sa[lr];
        const uint32_t z = s_z[lr];
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const int32_t c = (int32_t)((uint32_t)acc[t][j][r] - (uint32_t)csn[j] * z);
          const float f = (float)c;
          const float scl = swn[j] * s_a;
          float y = f * scl;
          y = y + bn[j];
          if (e.act == 1) y = bnh_silu_f32_t(y, s_tbl);
          else if (e.act == 2) y = bnh_relu_f32(y);
          T[(4 * (lane >> 4) + r) * TS + 16 * j + (lane & 15)] = y;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // lane: quad (lane % 32) of rows 2 it + lane / 32
      const int qd = lane & 31;
      float4 rq[8];
      if (RES) {  // every residual quad of the tile before any store (out and res may alias)
#pragma unroll
        for (int it = 0; it < 8; it++) {
          const int rr = 2 * it + (lane >> 5), lr = wm * 64 + 16 * t + rr;
          rq[it] = qd < nq && rowB + lr < rows
                       ? *(const float4 *)(e.res + s_r[lr] + n0 + wn * 128 + 4 * qd)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
#pragma unroll
      for (int it = 0; it < 8; it++) {
        const int rr = 2 * it + (lane >> 5), lr = wm * 64 + 16 * t + rr;
        if (qd < nq && rowB + lr < rows) {
          float4 y = *(const float4 *)(T + rr * TS + 4 * qd);
          if (RES) {
            y.x = y.x + rq[it].x;
            y.y = y.y + rq[it].y;
            y.z = y.z + rq[it].z;
            y.w = y.w + rq[it].w;
          }
          *(float4 *)(e.out + s_o[lr] + n0 + wn * 128 + 4 * qd) = y;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < 4; t++) {
    // the tile's residuals first (out and res may alias: every load of the tile before its stores)
    float rv[4][8];
    if (RES) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int lr = wm * 64 + 16 * t + 4 * (lane >> 4) + r;
        const float *rrow = e.res + s_r[lr];
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const int n = n0 + wn * 128 + 16 * j + (lane & 15);
          rv[r][j] = n < Np && rowB + lr < rows ? rrow[n] : 0.f;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int lr = wm * 64 + 16 * t + 4 * (lane >> 4) + r;
      if (rowB + lr >= rows) continue;
      const float s_a = s_sa[lr];
      const uint32_t z = s_z[lr];
      float *orow = e.out + s_o[lr];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int n = n0 + wn * 128 + 16 * j + (lane & 15);
        if (n >= Np) continue;
        const int32_t c = (int32_t)((uint32_t)acc[t][j][r] - (uint32_t)csn[j] * z);
        const float f = (float)c;
        const float scl = swn[j] * s_a;
        float y = f * scl;
        y = y + bn[j];
        if (e.act == 1) y = bnh_silu_f32_t(y, s_tbl);
        else if (e.act == 2) y = bnh_relu_f32(y);
        if (RES) y = y + rv[r][j];
        orow[n] = y;
      }
    }
  }
}

// ------------------------------------------------------------------ int8 GEMM, Q31 requant, NCHW
// A operand = x^T (pixels x K): x [K][M] has pixels contiguous, so each block stages a 64 k x 64 pixel tile through
// LDS transposed to [pixel][k] (4 x 4 byte blocks transposed in registers with v_perm), from where lane l reads its
// 16 k bytes of pixel (l & 15). B operand = w [Nt][K] rows straight from global (L2-resident).
// Accumulator lane layout: 4 consecutive pixels x 1 channel -> one 32-bit store of 4 output bytes.

#define RQ_LDS_STRIDE 80  // bytes per staged pixel row: 64 k + 16 pad

// Version 2: a block owns 128 pixels x 256 channels, so every activation byte is fetched from HBM once and every
// staged k row is one whole 128-byte line. Both operands go through LDS (rows of 64 k bytes at an 80-byte stride:
// the 16 rows a ds_read_b128 serves land on 16 disjoint 4-bank groups), prefetched into registers while the MFMAs of
// the current step run. 4 waves as 2 (pixels) x 2 (channels), each 64 pixels x 128 channels = 4 x 8 MFMA tiles.
#define RQ2_PIX 128
#define RQ2_CH 256
#define RQ2_LDS (RQ2_PIX * RQ_LDS_STRIDE + RQ2_CH * RQ_LDS_STRIDE)
__global__ __launch_bounds__(256, 2) void k_gemm_s8_requant2(const int8_t *__restrict__ x, long long x_ws, int M, int K,
                                                          int tiles_per_window, const int8_t *__restrict__ wt, int ldw,
                                                          const int32_t *__restrict__ bias_eff,
                                                          const int32_t *__restrict__ mult,
                                                          const int32_t *__restrict__ shift, int N, int zy, int lo,
                                                          int hi, int8_t *__restrict__ out, long long out_ws) {
  __shared__ __attribute__((aligned(16))) int8_t lds[2][RQ2_LDS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int win = blockIdx.x / tiles_per_window;
  const int p0 = (blockIdx.x % tiles_per_window) * RQ2_PIX;
  const int n0 = blockIdx.y * RQ2_CH;
  const int8_t *xw = x + win * x_ws;
  // activation staging: pixel quad pq (32 of them: one 128-byte line per k row), k quads kq and kq + 8
  const int pq = tid & 31, kq = tid >> 5;
  const int px = p0 + 4 * pq;
  const bool pin = px < M;  // M % 4 == 0
  // weight staging: channel row n0 + tid, 64 k bytes as 4 x 16
  const int8_t *wrow = wt + (long long)(n0 + tid) * ldw;
  const int kc = (lane >> 4) * 16;
  uint32_t rx[2][4];
  v4i rw[4];
  auto fetch = [&](int k0) {  // K % 16 == 0: a 4-row quad, a 16-byte weight chunk is all in or all out
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int k = k0 + 4 * (kq + 8 * h);
      const bool in = pin && k < K;
      const int8_t *src = xw + (long long)(in ? k : 0) * M + (in ? px : 0);
#pragma unroll
      for (int i = 0; i < 4; i++) rx[h][i] = *(const uint32_t *)(src + (in ? (long long)i * M : 0));
      if (!in) rx[h][0] = rx[h][1] = rx[h][2] = rx[h][3] = 0u;
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const bool in = k0 + 16 * c < K;
      rw[c] = *(const v4i *)(wrow + (in ? k0 + 16 * c : 0));
      if (!in) rw[c] = (v4i){0, 0, 0, 0};
    }
  };
  auto stage = [&](int8_t *buf) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      uint32_t c[4];
      transpose4x4(rx[h][0], rx[h][1], rx[h][2], rx[h][3], c);
#pragma unroll
      for (int j = 0; j < 4; j++) *(uint32_t *)(buf + (4 * pq + j) * RQ_LDS_STRIDE + 4 * (kq + 8 * h)) = c[j];
    }
    int8_t *wb = buf + RQ2_PIX * RQ_LDS_STRIDE + tid * RQ_LDS_STRIDE;
#pragma unroll
    for (int c = 0; c < 4; c++) *(v4i *)(wb + 16 * c) = rw[c];
  };
  v4i acc[4][8];
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int j = 0; j < 8; j++) acc[t][j] = (v4i){0, 0, 0, 0};
  fetch(0);
  stage(lds[0]);
  __syncthreads();
  int cur = 0;
  for (int k0 = 0; k0 < K; k0 += 64) {
    const bool more = k0 + 64 < K;
    if (more) fetch(k0 + 64);  // in flight during this step's MFMAs
    const int8_t *xs = lds[cur], *ws = lds[cur] + RQ2_PIX * RQ_LDS_STRIDE;
    v4i a[4];
#pragma unroll
    for (int t = 0; t < 4; t++) a[t] = *(const v4i *)(xs + (wm * 64 + 16 * t + (lane & 15)) * RQ_LDS_STRIDE + kc);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const v4i b = *(const v4i *)(ws + (wn * 128 + 16 * j + (lane & 15)) * RQ_LDS_STRIDE + kc);
#pragma unroll
      for (int t = 0; t < 4; t++) acc[t][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b, acc[t][j], 0, 0, 0);
    }
    if (more) {
      stage(lds[cur ^ 1]);  // the other buffer: last read two steps ago, before the previous barrier
      __syncthreads();
      cur ^= 1;
    }
  }
  int8_t *ow = out + win * out_ws;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int n = n0 + wn * 128 + 16 * j + (lane & 15);
    if (n >= N) continue;
    const int32_t be = bias_eff[n], mu = mult[n], sh = shift[n];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const int p = p0 + wm * 64 + 16 * t + 4 * (lane >> 4);
      if (p >= M) continue;
      uint32_t word = 0;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int32_t a32 = (int32_t)((uint32_t)acc[t][j][r] + (uint32_t)be);
        word |= ((uint32_t)bnh_requant(a32, mu, sh, zy, lo, hi) & 0xffu) << (8 * r);
      }
      *(uint32_t *)(ow + (long long)n * M + p) = word;
    }
  }
}

// Version 4 (M % 16 == 0): persistent blocks of 8 waves, one per CU. A tile is 256 pixels x 256 channels of one
// window (waves 4 (pixels) x 2 (channels), 64 x 128 each); a block walks its tiles t = blockIdx.x, + gridDim.x, ...,
// and the K steps of all its tiles form one 4-stage LDS ring fed by direct global -> LDS loads
// (global_load_lds_dwordx4: no registers, no VALU), so a tile's epilogue runs while the next tile's first steps load.
// Each block starts its K loop at its own step (K-step s + rot modulo the step count: the int32 sums are exact in any
// order), which spreads the blocks' weight-slice reads over L2.
//
// The activations stay in their k-major order in LDS; ds_read_b64_tr_b8 transposes them on the way to the MFMA
// operand: over a 16-lane group, output lane l byte b comes from the 8-byte chunk of source lane 2b + l/8, byte l % 8.
// Source lane j therefore points at k row 8h + j/2, pixels 8 (j % 2) .. + 7 of a 16-pixel column, and lane l receives
// pixel l's 8 k bytes of that half. XOR-swizzled 16-byte slots keep the DMA writes (64 consecutive slots per
// instruction) and the fragment reads free of bank conflicts:
//   activations: k row r (256 bytes), pixel column c (16 bytes) at r * 256 + 16 (c ^ (r & 7));
//   weights:     channel row n (64 bytes), k chunk c (16 bytes) at n * 64 + 16 (c ^ ((n >> 1) & 3)).
// K is padded to a multiple of 64 with zero weights (activation rows past K are clamped to row K - 1: multiplied by
// zero); pixel columns past M are clamped to the last column and their results dropped. The output tile is staged,
// 128 channels at a time, in the stage the last K step used and written as whole 256-byte channel rows.
#define RQ4_PIX 256
#define RQ4_CH 256
#define RQ4_BK 64
#define RQ4_XB (RQ4_BK * RQ4_PIX)
#define RQ4_STAGE (RQ4_XB + RQ4_CH * RQ4_BK)
#define RQ4_NST 4
#define RQ4_NLD 4  // DMA instructions per wave per K step: 2 activation + 2 weight
#define RQ4_MAXNT 1024  // channels (padded) whose requant vectors the kernel keeps in LDS
typedef int v2i __attribute__((ext_vector_type(2)));
// (direct global -> LDS loads: bnh_lds_dma.h)

__global__ __launch_bounds__(512, 1) void k_gemm_s8_requant4(const int8_t *__restrict__ x, long long x_ws, int M, int K,
                                                          int Kt, int tpw, int nblk, int ntiles,
                                                          const int8_t *__restrict__ wt,
                                                          const int32_t *__restrict__ bias_eff,
                                                          const int32_t *__restrict__ mult,
                                                          const int32_t *__restrict__ shift, int N, int zy, int lo,
                                                          int hi, int8_t *__restrict__ out, long long out_ws) {
  __shared__ __attribute__((aligned(1024))) int8_t lds_raw[RQ4_NST * RQ4_STAGE];
  // the per-channel requant vectors of all Nt channels (bias_eff, mult, shift), read by the epilogues from LDS: a
  // global load there would make the compiler wait for every DMA in flight (it counts only its own loads)
  __shared__ int32_t s_chan[3 * RQ4_MAXNT];
  lds_i8 *lds = (lds_i8 *)lds_raw;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int steps = Kt / RQ4_BK;
  for (int i = tid; i < nblk * RQ4_CH; i += 512) {
    s_chan[i] = bias_eff[i];
    s_chan[RQ4_MAXNT + i] = mult[i];
    s_chan[2 * RQ4_MAXNT + i] = shift[i];
  }
  __syncthreads();
  const int rot = (int)(blockIdx.x % steps);
  const int mytiles = ntiles > (int)blockIdx.x ? (ntiles - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  const int total = mytiles * steps;
  // tile t: channel block t % nblk, pixel tile (t / nblk) % tpw, window t / (nblk tpw)
  // DMA sources: activation instruction q (2 per wave) fills k rows 4q .. 4q + 3, lane -> row 4q + lane / 16, slot
  // lane % 16 = column (lane % 16) ^ (row % 8); weight instruction q (2 per wave) fills channel rows 16q .. 16q + 15,
  // lane -> row 16q + lane / 4, slot lane % 4 = chunk (lane % 4) ^ ((lane / 8) % 4)
  const int xr = lane >> 4, xslot = lane & 15;
  const int wrow = lane >> 2, wchunk = (lane & 3) ^ ((lane >> 3) & 3);
  // whole tiles (K % 64 == 0, M % 256 == 0): no row or column clamps, so each lane's offsets from the step's base
  // are the same at every step and the DMA takes its base in SGPRs
  const bool whole = K % RQ4_BK == 0 && M % RQ4_PIX == 0;
  uint32_t xoff[2], woff[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int q = 2 * wave + h, row = 4 * q + xr;
    xoff[h] = (uint32_t)(row * M + 16 * (xslot ^ (row & 7)));
    woff[h] = (uint32_t)((16 * q + wrow) * Kt + 16 * wchunk);
  }
  auto issue = [&](int gs) {
    const int t = (int)blockIdx.x + (gs / steps) * (int)gridDim.x;
    int s = gs % steps + rot;
    if (s >= steps) s -= steps;
    const int cb = t % nblk, rest = t / nblk, p0 = (rest % tpw) * RQ4_PIX, win = rest / tpw;
    const int8_t *xw = x + win * x_ws;
    lds_i8 *st = lds + (gs % RQ4_NST) * RQ4_STAGE;
    if (whole) {
      const int8_t *xb = xw + (long long)s * RQ4_BK * M + p0, *wb = wt + (long long)cb * RQ4_CH * Kt + s * RQ4_BK;
#pragma unroll
      for (int h = 0; h < 2; h++) rq_dma16s(xb, xoff[h], st + (2 * wave + h) * 1024);
#pragma unroll
      for (int h = 0; h < 2; h++) rq_dma16s(wb, woff[h], st + RQ4_XB + (2 * wave + h) * 1024);
      return;
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int q = 2 * wave + h, row = 4 * q + xr;
      int k = s * RQ4_BK + row;
      if (k > K - 1) k = K - 1;
      int px = p0 + 16 * (xslot ^ (row & 7));
      if (px > M - 16) px = M - 16;
      rq_dma16(xw + (long long)k * M + px, st + q * 1024);
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int q = 2 * wave + h;
      rq_dma16(wt + (long long)(cb * RQ4_CH + 16 * q + wrow) * Kt + s * RQ4_BK + 16 * wchunk, st + RQ4_XB + q * 1024);
    }
  };
  // fragment read offsets within a stage
  const int g = lane >> 4, j = lane & 15;
  int aoff[4][2], boff[8];
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      const int r = 16 * g + 8 * hf + (j >> 1), c = 4 * wm + t;
      aoff[t][hf] = r * RQ4_PIX + 16 * (c ^ (j >> 1)) + 8 * (j & 1);
    }
#pragma unroll
  for (int jj = 0; jj < 8; jj++) {
    const int n = wn * 128 + 16 * jj + j;
    boff[jj] = RQ4_XB + n * 64 + 16 * (g ^ ((n >> 1) & 3));
  }
  v4i acc[4][8];
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int jj = 0; jj < 8; jj++) acc[t][jj] = (v4i){0, 0, 0, 0};
  for (int gs = 0; gs < RQ4_NST - 1 && gs < total; gs++) issue(gs);
  for (int gs = 0; gs < total; gs++) {
    // this wave's loads of step gs have landed once at most the RQ4_NLD loads of each of the RQ4_NST - 2 later steps
    // are outstanding (loads retire in issue order; the count leaves out the epilogue's stores, which may retire
    // before older loads, so a pending store only lengthens the wait)
    if (gs + RQ4_NST - 2 >= total) RQ_WAIT_VM(0);
    else RQ_WAIT_VM(8);  // RQ4_NLD * (RQ4_NST - 2)
    RQ_BARRIER();  // every wave's loads of step gs have landed; the stage step gs - 1 used is no longer read
    if (gs + RQ4_NST - 1 < total) issue(gs + RQ4_NST - 1);
    const lds_i8 *st = lds + (gs % RQ4_NST) * RQ4_STAGE;
    v4i a[4], b[8];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const v2i lo8 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i *)(st + aoff[t][0]));
      const v2i hi8 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i *)(st + aoff[t][1]));
      a[t] = (v4i){lo8.x, lo8.y, hi8.x, hi8.y};
    }
#pragma unroll
    for (int jj = 0; jj < 8; jj++) b[jj] = *(const __attribute__((address_space(3))) v4i *)(st + boff[jj]);
#pragma unroll
    for (int jj = 0; jj < 8; jj++)
#pragma unroll
      for (int t = 0; t < 4; t++) acc[t][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[jj], acc[t][jj], 0, 0, 0);
    if (gs % steps != steps - 1) continue;
    // ---- epilogue of tile t: requantise, stage 128 channels x 256 pixels at a time, store whole rows
    const int t = (int)blockIdx.x + (gs / steps) * (int)gridDim.x;
    const int cb = t % nblk, rest = t / nblk, p0 = (rest % tpw) * RQ4_PIX, win = rest / tpw;
    // the window's output as a buffer: a store past it (channels >= N, pixels >= M) is dropped by the range check,
    // so every wave issues the same 8 store instructions
    const __amdgpu_buffer_rsrc_t orr =
        __builtin_amdgcn_make_buffer_rsrc((void *)(out + win * out_ws), 0, N * M, 0x00020000);
    uint32_t wd[8][4];
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      const int n = cb * RQ4_CH + wn * 128 + 16 * jj + j;  // < Nt: the per-channel vectors are padded to Nt
      const int32_t be = s_chan[n], mu = s_chan[RQ4_MAXNT + n], sh = s_chan[2 * RQ4_MAXNT + n];
      const bool s1 = sh >= 1 && sh <= 31;
      const BnhRqS1 rc = bnh_rq_s1(s1 ? sh : 1);
#pragma unroll
      for (int tt = 0; tt < 4; tt++) {
        uint32_t word = 0;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int32_t a32 = (int32_t)((uint32_t)acc[tt][jj][r] + (uint32_t)be);
          const int32_t y = s1 ? bnh_requant_s1(a32, mu, rc, zy, lo, hi) : bnh_requant(a32, mu, sh, zy, lo, hi);
          word |= ((uint32_t)y & 0xffu) << (8 * r);
        }
        wd[jj][tt] = word;
        acc[tt][jj] = (v4i){0, 0, 0, 0};
      }
    }
    // channel row ch (256 bytes) of the staging buffer holds 16-byte chunk c at ch * 256 + 16 (c ^ (ch & 15))
    lds_i8 *ob = lds + (gs % RQ4_NST) * RQ4_STAGE;
    RQ_BARRIER();  // every wave's MFMAs of step gs have read the stage
#pragma unroll
    for (int half = 0; half < 2; half++) {
      if (wn == half) {
#pragma unroll
        for (int jj = 0; jj < 8; jj++)
#pragma unroll
          for (int tt = 0; tt < 4; tt++) {
            const int ch = 16 * jj + j, px = wm * 64 + 16 * tt + 4 * g;
            *(__attribute__((address_space(3))) uint32_t *)(ob + ch * 256 + 16 * ((px >> 4) ^ (ch & 15)) + (px & 15)) =
                wd[jj][tt];
          }
      }
      RQ_BARRIER();
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int chunk = i * 512 + tid, ch = chunk >> 4, cp = chunk & 15;
        const v4i val = *(const __attribute__((address_space(3))) v4i *)(ob + ch * 256 + 16 * cp);
        const int n = cb * RQ4_CH + half * 128 + ch, p = p0 + 16 * (cp ^ (ch & 15));
        __builtin_amdgcn_raw_buffer_store_b128(val, orr, n < N && p < M ? n * M + p : 0x7ffffff0, 0, 0);
      }
      RQ_BARRIER();
    }
  }
}

// Version 5 (M % 16 == 0, 16-byte aligned output rows): the tiles, ring, LDS layouts and DMA roles of version 4,
// with the 8 waves in two ping-pong groups. Waves 0-3 (group 0) and 4-7 (group 1) put one wave of each group on every
// SIMD; the wave of group g owns pixels 128 g + 64 ((wave % 4) / 2) .. + 63 x channels 128 (wave % 2) .. + 127 of the
// tile. Each K step is a memory phase (the DMA three steps ahead, the step's 12 fragments into registers) then a
// compute phase (32 MFMAs), with a block barrier after each phase; group 1 starts one barrier late, so one group's
// fragment reads and waits overlap the other group's MFMAs. Step s is read by group 0 in interval 2s and by group 1
// in interval 2s + 1; the DMA of step s + 3 (issued in interval 2s or 2s + 1) refills the stage of step s - 1, last
// read in interval 2s - 1; every wave waits for its DMA of step s + 1 (vmcnt, counting only the loads issued after
// it) before the barrier that opens interval 2s + 2.
//   A tile's epilogue runs in the memory phase after its last compute phase and touches no LDS but the channel
// vectors: the 128 sums are requantised into 32 words (4 pixels each), a 4 x 4 word transpose across the lanes of
// each channel (permlane swaps) gives every lane 16 consecutive pixels of one channel, and each wave stores 8 x 16
// bytes per lane, 64 contiguous bytes per channel row.
BNH_DEV void rq_sync() {
  __builtin_amdgcn_sched_barrier(0);
  RQ_BARRIER();
  __builtin_amdgcn_sched_barrier(0);
}
// this wave's DMA of step s + 1 has landed: at most the loads of the (up to two) steps issued after it are pending
BNH_DEV void rq_wait_next(int total, int s) {
  const int later = total - 2 - s;
  if (later >= 2) RQ_WAIT_VM(8);
  else if (later == 1) RQ_WAIT_VM(4);
  else RQ_WAIT_VM(0);
}
// w[t] of lane (c, q) (c = lane % 16, q = lane / 16) -> w[i] of lane (c, q) = the old w[q] of lane (c, i)
BNH_DEV void rq_transpose_rows(uint32_t w[4]) {
  const auto p = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);  // rows 2, 3 of w0 <-> rows 0, 1 of w2
  const auto q = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
  const auto r = __builtin_amdgcn_permlane16_swap(p[0], q[0], false, false);  // rows 1, 3 of w0 <-> rows 0, 2 of w1
  const auto u = __builtin_amdgcn_permlane16_swap(p[1], q[1], false, false);
  w[0] = r[0];
  w[1] = r[1];
  w[2] = u[0];
  w[3] = u[1];
}

template <bool ALL_S1>  // every channel's shift is in 1..31
__global__ __launch_bounds__(512, 1) void k_gemm_s8_requant_pp(const int8_t *__restrict__ x, long long x_ws, int M,
                                                              int K, int Kt, int tpw, int nblk, int ntiles,
                                                              const int8_t *__restrict__ wt,
                                                              const int32_t *__restrict__ bias_eff,
                                                              const int32_t *__restrict__ mult,
                                                              const int32_t *__restrict__ shift, int N, int zy, int lo,
                                                              int hi, int8_t *__restrict__ out, long long out_ws) {
  __shared__ __attribute__((aligned(1024))) int8_t lds_raw[RQ4_NST * RQ4_STAGE];
  __shared__ int32_t s_chan[3 * RQ4_MAXNT];
  lds_i8 *lds = (lds_i8 *)lds_raw;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, wm = 2 * grp + ((wave & 3) >> 1), wn = wave & 1;
  const int steps = Kt / RQ4_BK;
  for (int i = tid; i < nblk * RQ4_CH; i += 512) {
    s_chan[i] = bias_eff[i];
    s_chan[RQ4_MAXNT + i] = mult[i];
    s_chan[2 * RQ4_MAXNT + i] = shift[i];
  }
  __syncthreads();
  const int rot = (int)(blockIdx.x % steps);
  const int mytiles = ntiles > (int)blockIdx.x ? (ntiles - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  const int total = mytiles * steps;
  const int xr = lane >> 4, xslot = lane & 15;
  const int wrow = lane >> 2, wchunk = (lane & 3) ^ ((lane >> 3) & 3);
  const bool whole = K % RQ4_BK == 0 && M % RQ4_PIX == 0;
  uint32_t xoff[2], woff[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int q = 2 * wave + h, row = 4 * q + xr;
    xoff[h] = (uint32_t)(row * M + 16 * (xslot ^ (row & 7)));
    woff[h] = (uint32_t)((16 * q + wrow) * Kt + 16 * wchunk);
  }
  int iss = 0;  // the next step to issue
  auto issue = [&]() {
    const int gs = iss++;
    const int t = (int)blockIdx.x + (gs / steps) * (int)gridDim.x;
    int s = gs % steps + rot;
    if (s >= steps) s -= steps;
    const int cb = t % nblk, rest = t / nblk, p0 = (rest % tpw) * RQ4_PIX, win = rest / tpw;
    const int8_t *xw = x + win * x_ws;
    lds_i8 *st = lds + (gs % RQ4_NST) * RQ4_STAGE;
    if (whole) {
      const int8_t *xb = xw + (long long)s * RQ4_BK * M + p0, *wb = wt + (long long)cb * RQ4_CH * Kt + s * RQ4_BK;
#pragma unroll
      for (int h = 0; h < 2; h++) rq_dma16s(xb, xoff[h], st + (2 * wave + h) * 1024);
#pragma unroll
      for (int h = 0; h < 2; h++) rq_dma16s(wb, woff[h], st + RQ4_XB + (2 * wave + h) * 1024);
      return;
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int q = 2 * wave + h, row = 4 * q + xr;
      int k = s * RQ4_BK + row;
      if (k > K - 1) k = K - 1;
      int px = p0 + 16 * (xslot ^ (row & 7));
      if (px > M - 16) px = M - 16;
      rq_dma16(xw + (long long)k * M + px, st + q * 1024);
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int q = 2 * wave + h;
      rq_dma16(wt + (long long)(cb * RQ4_CH + 16 * q + wrow) * Kt + s * RQ4_BK + 16 * wchunk, st + RQ4_XB + q * 1024);
    }
  };
  const int g = lane >> 4, j = lane & 15;
  int aoff[4][2], boff[8];
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      const int r = 16 * g + 8 * hf + (j >> 1), c = 4 * wm + t;
      aoff[t][hf] = r * RQ4_PIX + 16 * (c ^ (j >> 1)) + 8 * (j & 1);
    }
#pragma unroll
  for (int jj = 0; jj < 8; jj++) {
    const int n = wn * 128 + 16 * jj + j;
    boff[jj] = RQ4_XB + n * 64 + 16 * (g ^ ((n >> 1) & 3));
  }
  v4i acc[4][8];
  // tile i's outputs: acc[tt][jj][r] is pixel wm 64 + 16 tt + 4 g + r, channel wn 128 + 16 jj + j of the tile
  auto epilogue = [&](int i) {
    const int t = (int)blockIdx.x + i * (int)gridDim.x;
    const int cb = t % nblk, rest = t / nblk, p0 = (rest % tpw) * RQ4_PIX, win = rest / tpw;
    // the window's output as a buffer: stores past it are dropped, so every wave issues the same 8 stores
    const __amdgpu_buffer_rsrc_t orr =
        __builtin_amdgcn_make_buffer_rsrc((void *)(out + win * out_ws), 0, N * M, 0x00020000);
    const int p = p0 + wm * 64 + 16 * g;  // this lane's 16 pixels after the transpose
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      const int nl = wn * 128 + 16 * jj + j, n = cb * RQ4_CH + nl;  // < Nt: the channel vectors are padded to Nt
      const int32_t be = s_chan[n], mu = s_chan[RQ4_MAXNT + n], sh = s_chan[2 * RQ4_MAXNT + n];
      const bool s1 = ALL_S1 || (sh >= 1 && sh <= 31);
      const BnhRqS1 rc = bnh_rq_s1(s1 ? sh : 1);
      uint32_t w[4];
#pragma unroll
      for (int tt = 0; tt < 4; tt++) {
        uint32_t word = 0;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int32_t a32 = (int32_t)((uint32_t)acc[tt][jj][r] + (uint32_t)be);
          const int32_t y = s1 ? bnh_requant_s1(a32, mu, rc, zy, lo, hi) : bnh_requant(a32, mu, sh, zy, lo, hi);
          word |= ((uint32_t)y & 0xffu) << (8 * r);
        }
        w[tt] = word;
      }
      rq_transpose_rows(w);
      const v4i val = (v4i){(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
      __builtin_amdgcn_raw_buffer_store_b128(val, orr, n < N && p < M ? n * M + p : 0x7ffffff0, 0, 0);
    }
  };
  for (int s = 0; s < RQ4_NST - 1 && s < total; s++) issue();
  if (total > 2) RQ_WAIT_VM(8);  // step 0 has landed
  else if (total == 2) RQ_WAIT_VM(4);
  else RQ_WAIT_VM(0);
  rq_sync();
  if (grp) rq_sync();  // group 1 runs one phase behind group 0
  int ck = 0, ci = 0, done = -1;
  for (int s = 0; s < total; s++) {
    asm volatile("" : "+s"(done));  // opaque to the optimiser: no peeled first iteration
    // ---- memory phase of step s
    if (s + RQ4_NST - 1 < total) issue();
    if (done >= 0) {
      epilogue(done);
      done = -1;
    }
    const lds_i8 *st = lds + (s % RQ4_NST) * RQ4_STAGE;
    v4i a[4], b[8];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const v2i lo8 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i *)(st + aoff[t][0]));
      const v2i hi8 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i *)(st + aoff[t][1]));
      a[t] = (v4i){lo8.x, lo8.y, hi8.x, hi8.y};
    }
#pragma unroll
    for (int jj = 0; jj < 8; jj++) b[jj] = *(const __attribute__((address_space(3))) v4i *)(st + boff[jj]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (grp) rq_wait_next(total, s);
    rq_sync();
    // ---- compute phase of step s (a tile's first step starts its sums from zero)
    if (ck == 0) {
#pragma unroll
      for (int jj = 0; jj < 8; jj++)
#pragma unroll
        for (int t = 0; t < 4; t++)
          acc[t][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[jj], (v4i){0, 0, 0, 0}, 0, 0, 0);
    } else {
#pragma unroll
      for (int jj = 0; jj < 8; jj++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[t][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[jj], acc[t][jj], 0, 0, 0);
    }
    if (++ck == steps) {
      done = ci;
      ck = 0;
      ci++;
    }
    if (!grp) rq_wait_next(total, s);
    rq_sync();
  }
  if (done >= 0) epilogue(done);
  if (!grp) rq_sync();  // every wave passes the same number of barriers
}

// Version 6 (split rings): version 5's tiles, wave roles, phases and epilogue, with the activations and the weights
// in LDS rings of their own, each filled by one group: group 0 (waves 0-3) issues the activation DMA XST - 1 steps
// ahead, group 1 (waves 4-7) the weight DMA WST - 1 steps ahead. A wave's vmcnt counts only its own loads, so the
// weight loads (L2 hits) never hold up an activation wait, and XST stages of 16 KB keep (XST - 1) x 16 KB of HBM reads
// in flight per CU where version 5's shared ring holds 3 x 16 KB.
//   Step s is read by group 0 in interval 2s and by group 1 in interval 2s + 1. The activation DMA of step s + XST - 1
// (group 0, interval 2s) refills the stage of step s - 1, last read in interval 2s - 1; the weight DMA of step
// s + WST - 1 (group 1, interval 2s + 1) refills the stage of step s - 1 as well (WST >= 3: the weights of step s + 1
// are read in interval 2s + 2). Each wave waits for its own DMA of step s + 1 before the barrier that opens interval
// 2s + 2; a wave's epilogue stores are counted by the same vmcnt and can only lengthen that wait.
//   Measured at 1152 -> 256 channels over 1536 pixels x 256 windows, deeper activation rings (6 + 3, 5 + 4 stages) ran
// slower than 4 + 4, so the launcher instantiates 4 + 4.
//   The short epilogue (EPI 2, bnh_q8w::fast) needs no sign test: when zy <= lo a negative product requantises to
// lo under either rounding of its sign, so every output is zy + clamp(hi32(acc mult + cq) >> e1, lo - zy, hi - zy)
// (one 64-bit multiply-add, a shift and a median per output; zy added to four packed bytes at once), about 5 VALU
// instructions per output where the general form takes about 12.
#define RQ6_SB 16384  // one stage of either ring: 64 k rows x 256 pixels, or 256 channels x 64 k
template <int N>
BNH_DEV void rq_wait_vm_steps(int later) {  // at most `later` steps of N loads each outstanding (later in 0..4)
  static_assert(N == 4, "four DMA instructions per wave and step");
  if (later >= 4) RQ_WAIT_VM(16);
  else if (later == 3) RQ_WAIT_VM(12);
  else if (later == 2) RQ_WAIT_VM(8);
  else if (later == 1) RQ_WAIT_VM(4);
  else RQ_WAIT_VM(0);
}

template <int EPI, int XST, int WST>  // EPI: 0 any shift, 1 shifts 1..31, 2 the short epilogue (bnh_q8w::fast)
__global__ __launch_bounds__(512, 1) void k_gemm_s8_requant_sr(const int8_t *__restrict__ x, long long x_ws, int M,
                                                              int K, int Kt, int tpw, int nblk, int ntiles,
                                                              const int8_t *__restrict__ wt,
                                                              const int32_t *__restrict__ bias_eff,
                                                              const int32_t *__restrict__ mult,
                                                              const int32_t *__restrict__ shift, int N, int zy, int lo,
                                                              int hi, int8_t *__restrict__ out, long long out_ws,
                                                              const int32_t *__restrict__ cq,
                                                              const int32_t *__restrict__ e1v) {
  static_assert(WST >= 3 && XST >= 2 && XST - 2 <= 4 && WST - 2 <= 4, "ring depths");
  __shared__ __attribute__((aligned(1024))) int8_t lds_raw[(XST + WST) * RQ6_SB];
  __shared__ int32_t s_chan[4 * RQ4_MAXNT];
  lds_i8 *xlds = (lds_i8 *)lds_raw, *wlds = xlds + XST * RQ6_SB;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, wq = wave & 3, wm = 2 * grp + (wq >> 1), wn = wave & 1;
  const int steps = Kt / RQ4_BK;
  const int Nt = nblk * RQ4_CH;
  for (int i = tid; i < Nt; i += 512) {
    if (EPI == 2) {
      s_chan[i] = cq[i];
      s_chan[RQ4_MAXNT + i] = cq[Nt + i];
      s_chan[3 * RQ4_MAXNT + i] = e1v[i];
    } else {
      s_chan[i] = bias_eff[i];
      s_chan[3 * RQ4_MAXNT + i] = shift[i];
    }
    s_chan[2 * RQ4_MAXNT + i] = mult[i];
  }
  __syncthreads();
  const int rot = (int)(blockIdx.x % steps);
  const int mytiles = ntiles > (int)blockIdx.x ? (ntiles - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  const int total = mytiles * steps;
  // the short epilogue's output bytes: c = clamp(v, lo - zy, hi - zy) in 0..255, then c + zy in each byte of a word
  // of four (a carry-free bytewise add)
  const int lz = lo - zy, hz = hi - zy;
  const uint32_t zb = (uint32_t)(zy & 0xff) * 0x01010101u, zb7 = zb & 0x7f7f7f7fu;
  const int nst = grp ? WST : XST;  // this wave's ring
  // this wave's 4 DMA instructions of a step, q = 4 (wave % 4) + h. Group 0: activation instruction q fills k rows
  // 4q .. 4q + 3, lane -> row 4q + lane / 16, its 16-byte slot lane % 16 holding pixel column (lane % 16) ^ (row % 8).
  // Group 1: weight instruction q fills channel rows 16q .. 16q + 15, lane -> row 16q + lane / 4, its slot lane % 4
  // holding k chunk (lane % 4) ^ ((lane / 8) % 4).
  const int xr = lane >> 4, xslot = lane & 15;
  const int wrow = lane >> 2, wchunk = (lane & 3) ^ ((lane >> 3) & 3);
  const bool whole = K % RQ4_BK == 0 && M % RQ4_PIX == 0;
  uint32_t doff[4];
#pragma unroll
  for (int h = 0; h < 4; h++) {
    const int q = 4 * wq + h, row = 4 * q + xr;
    doff[h] = grp ? (uint32_t)((16 * q + wrow) * Kt + 16 * wchunk) : (uint32_t)(row * M + 16 * (xslot ^ (row & 7)));
  }
  int iss = 0;  // the next step this wave issues
  auto issue = [&]() {
    const int gs = iss++;
    const int t = (int)blockIdx.x + (gs / steps) * (int)gridDim.x;
    const int cb = t % nblk, rest = t / nblk, p0 = (rest % tpw) * RQ4_PIX, win = rest / tpw;
    int s = gs % steps + rot;
    if (s >= steps) s -= steps;
    if (grp) {  // weights: padded to Nt x Kt, never clamped
      lds_i8 *st = wlds + (gs % WST) * RQ6_SB;
      const int8_t *wb = wt + (long long)cb * RQ4_CH * Kt + s * RQ4_BK;
#pragma unroll
      for (int h = 0; h < 4; h++) rq_dma16s(wb, doff[h], st + (4 * wq + h) * 1024);
      return;
    }
    lds_i8 *st = xlds + (gs % XST) * RQ6_SB;
    const int8_t *xw = x + win * x_ws;
    if (whole) {
      const int8_t *xb = xw + (long long)s * RQ4_BK * M + p0;
#pragma unroll
      for (int h = 0; h < 4; h++) rq_dma16s_nt(xb, doff[h], st + (4 * wq + h) * 1024);  // read once: non-temporal
      return;
    }
#pragma unroll
    for (int h = 0; h < 4; h++) {
      const int q = 4 * wq + h, row = 4 * q + xr;
      int k = s * RQ4_BK + row;
      if (k > K - 1) k = K - 1;
      int px = p0 + 16 * (xslot ^ (row & 7));
      if (px > M - 16) px = M - 16;
      rq_dma16(xw + (long long)k * M + px, st + q * 1024);
    }
  };
  const int g = lane >> 4, j = lane & 15;
  int aoff[4][2], boff[8];
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      const int r = 16 * g + 8 * hf + (j >> 1), c = 4 * wm + t;
      aoff[t][hf] = r * RQ4_PIX + 16 * (c ^ (j >> 1)) + 8 * (j & 1);
    }
#pragma unroll
  for (int jj = 0; jj < 8; jj++) {
    const int n = wn * 128 + 16 * jj + j;
    boff[jj] = n * 64 + 16 * (g ^ ((n >> 1) & 3));
  }
  v4i acc[4][8];
  // tile i's outputs: acc[tt][jj][r] is pixel wm 64 + 16 tt + 4 g + r, channel wn 128 + 16 jj + j of the tile
  auto epilogue = [&](int i) {
    const int t = (int)blockIdx.x + i * (int)gridDim.x;
    const int cb = t % nblk, rest = t / nblk, p0 = (rest % tpw) * RQ4_PIX, win = rest / tpw;
    const __amdgpu_buffer_rsrc_t orr =
        __builtin_amdgcn_make_buffer_rsrc((void *)(out + win * out_ws), 0, N * M, 0x00020000);
    const int p = p0 + wm * 64 + 16 * g;  // this lane's 16 pixels after the transpose
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      const int nl = wn * 128 + 16 * jj + j, n = cb * RQ4_CH + nl;
      const int32_t mu = s_chan[2 * RQ4_MAXNT + n];
      uint32_t w[4];
      if (EPI == 2) {
        const int64_t c = (int64_t)(((uint64_t)(uint32_t)s_chan[RQ4_MAXNT + n] << 32) | (uint32_t)s_chan[n]);
        const int e1 = s_chan[3 * RQ4_MAXNT + n];
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
          uint32_t word = 0;
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int32_t v = (int32_t)(((int64_t)acc[tt][jj][r] * mu + c) >> 32) >> e1;
            int32_t cl;
            asm("v_med3_i32 %0, %1, %2, %3" : "=v"(cl) : "v"(v), "v"(lz), "v"(hz));
            word |= (uint32_t)cl << (8 * r);
          }
          w[tt] = ((word & 0x7f7f7f7fu) + zb7) ^ ((word ^ zb) & 0x80808080u);
        }
      } else {
        const int32_t be = s_chan[n], sh = s_chan[3 * RQ4_MAXNT + n];
        const bool s1 = EPI == 1 || (sh >= 1 && sh <= 31);
        const BnhRqS1 rc = bnh_rq_s1(s1 ? sh : 1);
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
          uint32_t word = 0;
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int32_t a32 = (int32_t)((uint32_t)acc[tt][jj][r] + (uint32_t)be);
            const int32_t y = s1 ? bnh_requant_s1(a32, mu, rc, zy, lo, hi) : bnh_requant(a32, mu, sh, zy, lo, hi);
            word |= ((uint32_t)y & 0xffu) << (8 * r);
          }
          w[tt] = word;
        }
      }
      rq_transpose_rows(w);
      const v4i val = (v4i){(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
      __builtin_amdgcn_raw_buffer_store_b128(val, orr, n < N && p < M ? n * M + p : 0x7ffffff0, 0, 0);
    }
  };
  // prologue: each group issues its ring's first nst - 1 steps and waits for step 0
  const int pre = nst - 1 < total ? nst - 1 : total;
  for (int s = 0; s < pre; s++) issue();
  if (pre > 0) rq_wait_vm_steps<4>(pre - 1);
  rq_sync();
  if (grp) rq_sync();  // group 1 runs one phase behind group 0
  int ck = 0, ci = 0, done = -1;
  for (int s = 0; s < total; s++) {
    asm volatile("" : "+s"(done));  // opaque to the optimiser: no peeled first iteration
    // ---- memory phase of step s
    if (s + nst - 1 < total) issue();
    if (done >= 0) {
      epilogue(done);
      done = -1;
    }
    const lds_i8 *xs = xlds + (s % XST) * RQ6_SB, *ws = wlds + (s % WST) * RQ6_SB;
    v4i a[4], b[8];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const v2i lo8 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i *)(xs + aoff[t][0]));
      const v2i hi8 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i *)(xs + aoff[t][1]));
      a[t] = (v4i){lo8.x, lo8.y, hi8.x, hi8.y};
    }
#pragma unroll
    for (int jj = 0; jj < 8; jj++) b[jj] = *(const __attribute__((address_space(3))) v4i *)(ws + boff[jj]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // this wave's DMA of step s + 1 has landed once at most the steps it issued after that one are outstanding
    const int later = (total - 2 - s < nst - 2 ? total - 2 - s : nst - 2);
    if (grp) rq_wait_vm_steps<4>(later);
    rq_sync();
    // ---- compute phase of step s (a tile's first step starts its sums from zero)
    if (ck == 0) {
#pragma unroll
      for (int jj = 0; jj < 8; jj++)
#pragma unroll
        for (int t = 0; t < 4; t++)
          acc[t][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[jj], (v4i){0, 0, 0, 0}, 0, 0, 0);
    } else {
#pragma unroll
      for (int jj = 0; jj < 8; jj++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[t][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[jj], acc[t][jj], 0, 0, 0);
    }
    if (++ck == steps) {
      done = ci;
      ck = 0;
      ci++;
    }
    if (!grp) rq_wait_vm_steps<4>(later);
    rq_sync();
  }
  if (done >= 0) epilogue(done);
  if (!grp) rq_sync();  // every wave passes the same number of barriers
}

// requant arithmetic check: y[i] = bnh_requant(acc[i], mult[i], shift[i], zy, lo, hi), where for shift 1..31 the
// one-rounding form must agree (INT32_MIN, outside every clamp range, marks a disagreement)
__global__ void k_eval_requant(const int32_t *__restrict__ acc, const int32_t *__restrict__ mult,
                               const int32_t *__restrict__ shift, int zy, int lo, int hi, int32_t *__restrict__ y,
                               long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t r = bnh_requant(acc[i], mult[i], shift[i], zy, lo, hi);
  const bool s1 = shift[i] >= 1 && shift[i] <= 31;
  y[i] = !s1 || bnh_requant_s1(acc[i], mult[i], bnh_rq_s1(shift[i]), zy, lo, hi) == r ? r : INT32_MIN;
}

// ------------------------------------------------------------------ numerics probe
// f: 0 FRECPE, 1 the SiLU of the epilogues (LDS-table form), 2 ReLU, 3 the SiLU without the table
__global__ void k_eval_f32(int f, const float *__restrict__ x, float *__restrict__ y, long long n) {
  __shared__ uint32_t tbl[256];
  bnh_silu_table(tbl);
  __syncthreads();
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  y[i] = f == 0 ? bnh_frecpe(v) : f == 1 ? bnh_silu_f32_t(v, tbl) : f == 3 ? bnh_silu_f32(v) : bnh_relu_f32(v);
}

// ================================================================== host side
extern "C" {

int bnh_eval_requant(const int32_t *acc, const int32_t *mult, const int32_t *shift, int zy, int lo, int hi, int32_t *y,
                     long long n, void *stream) {
  BNH_REQ(acc && mult && shift && y && n >= 0 && lo <= hi);
  if (!n) return 0;
  hipLaunchKernelGGL(k_eval_requant, dim3((unsigned)bnh_ceil_div(n, 256)), dim3(256), 0, bnh_stream(stream), acc, mult,
                     shift, zy, lo, hi, y, n);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_eval_f32(int f, const float *x, float *y, long long n, void *stream) {
  BNH_REQ(f >= 0 && f <= 3 && n >= 0 && x && y);
  if (!n) return 0;
  hipLaunchKernelGGL(k_eval_f32, dim3((unsigned)bnh_ceil_div(n, 256)), dim3(256), 0, bnh_stream(stream), f, x, y, n);
  BNH_HIP(hipGetLastError());
  return 0;
}

bnh_s8w *bnh_s8w_new(int N, int K, int Kp, int Np, const int8_t *w, const float *sw, const int32_t *colsum,
                     const float *b) {
  if (N <= 0 || K <= 0 || Np != ((N + 7) & ~7) || Kp != ((K + 15) & ~15) || !w || !sw || !colsum || !b) {
    bnh_fail("bnh_s8w_new: int8 GEMM shape N %d K %d Kp %d Np %d: expected Np = N rounded up to 8, Kp = K rounded "
             "up to 16, and all four tensors", N, K, Kp, Np);
    return nullptr;
  }
  const int Nt = (int)bnh_round_up(Np, 128);
  int8_t *hw = (int8_t *)calloc((size_t)Nt * Kp, 1);
  float *hsw = (float *)calloc(Nt, 4), *hb = (float *)calloc(Nt, 4);
  int32_t *hcs = (int32_t *)calloc(Nt, 4);
  bnh_s8w *W = (bnh_s8w *)calloc(1, sizeof *W);
  if (!hw || !hsw || !hb || !hcs || !W) {
    free(hw); free(hsw); free(hb); free(hcs); free(W);
    bnh_fail("bnh_s8w_new: out of host memory");
    return nullptr;
  }
  const int kb = Kp / 16;
  for (int n = 0; n < Np; n++)
    for (int k = 0; k < Kp; k++)
      hw[(size_t)n * Kp + k] = w[((size_t)(n / 4) * kb + k / 16) * 64 + (n % 4) * 16 + k % 16];
  memcpy(hsw, sw, sizeof(float) * Np);
  memcpy(hb, b, sizeof(float) * Np);
  memcpy(hcs, colsum, sizeof(int32_t) * Np);
  W->N = N; W->K = K; W->Kp = Kp; W->Np = Np; W->Nt = Nt;
  bool ok = (W->w = (int8_t *)bnh_malloc((size_t)Nt * Kp)) && (W->sw = (float *)bnh_malloc(4 * (size_t)Nt)) &&
            (W->b = (float *)bnh_malloc(4 * (size_t)Nt)) && (W->colsum = (int32_t *)bnh_malloc(4 * (size_t)Nt)) &&
            !bnh_memcpy_h2d(W->w, hw, (size_t)Nt * Kp) && !bnh_memcpy_h2d(W->sw, hsw, 4 * (size_t)Nt) &&
            !bnh_memcpy_h2d(W->b, hb, 4 * (size_t)Nt) && !bnh_memcpy_h2d(W->colsum, hcs, 4 * (size_t)Nt);
  free(hw); free(hsw); free(hb); free(hcs);
  if (!ok) { bnh_s8w_free(W); return nullptr; }
  return W;
}

void bnh_s8w_free(bnh_s8w *W) {
  if (!W) return;
  if (W->w) (void)hipFree(W->w);
  if (W->sw) (void)hipFree(W->sw);
  if (W->b) (void)hipFree(W->b);
  if (W->colsum) (void)hipFree(W->colsum);
  free(W);
}

int bnh_s8n_quant_rows(const float *x, long long x_ws, int ld, int M, int K, int Kp, const float *gate,
                       long long gate_ws, int8_t *q, long long q_ws, float *sa, long long sa_ws, int32_t *za,
                       long long za_ws, int B, void *stream) {
  BNH_REQ(x && q && sa && za && M > 0 && K > 0 && B > 0);
  BNH_REQ(Kp == ((K + 15) & ~15) && ld >= K);
  BNH_REQ(!gate || (K % 4 == 0 && K <= 4096));
  BNH_REQ(((uintptr_t)q & 3) == 0 && q_ws % 4 == 0 && (B == 1 || q_ws >= (long long)M * Kp));
  BNH_REQ(B == 1 || (x_ws >= (long long)(M - 1) * ld + K && sa_ws >= M && za_ws >= M));
  const long long rows = (long long)M * B;
  const bool vec = ((uintptr_t)x & 15) == 0 && ld % 4 == 0 && (B == 1 || x_ws % 4 == 0) &&
                   (!gate || (((uintptr_t)gate & 15) == 0 && (B == 1 || gate_ws % 4 == 0)));
  hipStream_t st = bnh_stream(stream);
  if (!vec) {
    hipLaunchKernelGGL(k_s8n_quant, dim3((unsigned)bnh_ceil_div(rows, 4)), dim3(256), 0, st, x, x_ws, ld, M, K, Kp,
                       gate, gate_ws, q, q_ws, sa, sa_ws, za, za_ws, rows);
  } else {
    int L = 1;  // about four 16-byte chunks of a row per lane
    while (L < 64 && 16 * L < Kp) L *= 2;
#define QV(LL)                                                                                                         \
  hipLaunchKernelGGL((k_s8n_quant_v<LL>), dim3((unsigned)bnh_ceil_div(rows, 256 / LL)), dim3(256), 0, st, x, x_ws, ld, \
                     M, K, Kp, gate, gate_ws, q, q_ws, sa, sa_ws, za, za_ws, rows, 1.0 / M)
    switch (L) {
      case 1: QV(1); break;
      case 2: QV(2); break;
      case 4: QV(4); break;
      case 8: QV(8); break;
      case 16: QV(16); break;
      case 32: QV(32); break;
      default: QV(64); break;
    }
#undef QV
  }
  BNH_HIP(hipGetLastError());
  return 0;
}

static int check_epi(const bnh_epi32 *e, int M, int Np, int B) {
  BNH_REQ(e && e->out && e->act >= 0 && e->act <= 2 && e->ldo >= Np);
  BNH_REQ(e->opad >= 0 && e->opad <= 3 && (!e->opad || (e->ow > 0 && M % e->ow == 0)));
  BNH_REQ(!e->res || (e->ldr >= Np && e->rpad >= 0 && (!e->rpad || (e->rw > 0 && M % e->rw == 0))));
  (void)B;
  return 0;
}

int bnh_s8n_gemm(const int8_t *q, long long q_ws, const float *sa, long long sa_ws, const int32_t *za, long long za_ws,
                 int M, int B, const bnh_s8w *W, const bnh_epi32 *e, void *stream) {
  BNH_REQ(q && sa && za && W && M > 0 && B > 0);
  BNH_REQ(((uintptr_t)q & 15) == 0 && q_ws % 16 == 0);
  if (check_epi(e, M, W->Np, B)) return -1;
  const long long rows = (long long)M * B;
  EpiDev d = {e->act, e->out, e->out_ws, e->ldo, e->ow, e->opad, e->res, e->res_ws, e->ldr, e->rpad, e->rw,
              e->opad ? 1.0 / e->ow : 0.0, e->rpad ? 1.0 / e->rw : 0.0, 0};
  // with a residual, 16-byte quads when every output and residual quad lies 16-byte aligned (block 1's 24 -> 24
  // projection over 249 x 63 pixels 341 -> 322 us; without a residual the quads' LDS round trip made the launches
  // 10-30 % slower, so those store values directly)
  auto al4 = [](const void *p, long long ws, int ld) { return ((uintptr_t)p & 15) == 0 && ws % 4 == 0 && ld % 4 == 0; };
  d.vec = W->Np % 4 == 0 && e->res && al4(e->out, e->out_ws, e->ldo) && al4(e->res, e->res_ws, e->ldr);
  hipStream_t s = bnh_stream(stream);
  const double rM = 1.0 / M;
  // 128 rows per block; the channel groups split over gsplit blocks only when the row blocks alone would leave the
  // chip short of blocks (fewer than 1024)
  const long long nrb = bnh_ceil_div(rows, 128);
  const int ng = (W->Np + 63) / 64;
  // large K with rows enough for 4 tiles per CU: the LDS-staged tile kernel (each row read once, fragment loads
  // pipelined; config 0's 1152 -> 256 over 393,216 rows: 0.70 -> 0.32 ms). Fewer rows (the Perch-shaped
  // projections, 16k-65k rows) keep the group-split kernel, which fills the chip with more, smaller blocks.
  const bool wide = W->Np > 128;  // 128 rows x 256 channels, else 256 rows x 128 channels
  const int TR = wide ? 128 : 256, TN = wide ? 256 : 128;
  const int nct = (int)bnh_ceil_div(W->Np, TN);
  const long long blocks = bnh_ceil_div(rows, TR) * nct;
  if (W->Kp >= 256 && blocks >= 1024) {
    // rows stored as 16-byte quads when every output (and residual) row start is 16-byte aligned
    d.vec = W->Np % 4 == 0 && al4(e->out, e->out_ws, e->ldo) && (!e->res || al4(e->res, e->res_ws, e->ldr));
    BNH_REQ(blocks < (1LL << 31));
#define S8N_LDS_LAUNCH(WM_, WN_, RES_)                                                                             \
  hipLaunchKernelGGL((k_s8n_gemm_lds<WM_, WN_, RES_>), dim3((unsigned)blocks), dim3(256), 0, s, q, q_ws, sa, sa_ws, za, \
                     za_ws, M, rM, rows, W->w, W->sw, W->colsum, W->b, W->Kp, W->Np, W->Nt, nct, d)
    if (wide && e->res) S8N_LDS_LAUNCH(2, 2, true);
    else if (wide) S8N_LDS_LAUNCH(2, 2, false);
    else if (e->res) S8N_LDS_LAUNCH(4, 1, true);
    else S8N_LDS_LAUNCH(4, 1, false);
#undef S8N_LDS_LAUNCH
    BNH_HIP(hipGetLastError());
    return 0;
  }
  int gsplit = 1;
  if (nrb < 1024) gsplit = (int)bnh_ceil_div(1024, nrb);
  if (gsplit > ng) gsplit = ng;
  BNH_REQ(nrb * gsplit < (1LL << 31));
  if (e->res)
    hipLaunchKernelGGL(k_s8n_gemm<true>, dim3((unsigned)(nrb * gsplit)), dim3(256), 0, s, q, q_ws, sa, sa_ws, za, za_ws,
                       M, rM, rows, W->w, W->sw, W->colsum, W->b, W->Kp, W->Np, gsplit, d);
  else
    hipLaunchKernelGGL(k_s8n_gemm<false>, dim3((unsigned)(nrb * gsplit)), dim3(256), 0, s, q, q_ws, sa, sa_ws, za,
                       za_ws, M, rM, rows, W->w, W->sw, W->colsum, W->b, W->Kp, W->Np, gsplit, d);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_pw_s8(const float *in, long long in_ws, int lda, int M, const float *gate, long long gate_ws, int8_t *q,
              long long q_ws, float *sa, long long sa_ws, int32_t *za, long long za_ws, int B, const bnh_s8w *W,
              const bnh_epi32 *e, void *stream) {
  BNH_REQ(W && e && e->out);
  if (check_epi(e, M, W->Np, B)) return -1;
  if (e->opad) {
    const int H = M / e->ow, Wd = e->ow, h = e->opad;
    const long long per = (long long)(H + 2 * h) * (Wd + 2 * h) * e->ldo;
    BNH_REQ(B == 1 || e->out_ws >= per);
    if (bnh_zero_halo(e->out, B == 1 ? per : e->out_ws, H, Wd, e->ldo, h, 4, B, stream)) return -1;
  }
  if (bnh_s8n_quant_rows(in, in_ws, lda, M, W->K, W->Kp, gate, gate_ws, q, q_ws, sa, sa_ws, za, za_ws, B, stream))
    return -1;
  return bnh_s8n_gemm(q, q_ws, sa, sa_ws, za, za_ws, M, B, W, e, stream);
}

bnh_q8w *bnh_q8w_new(int N, int K, const int8_t *w, const int32_t *bias, const int32_t *mult, const int32_t *shift,
                     int zx, int zy, int lo, int hi) {
  if (N <= 0 || K <= 0 || !w || !bias || !mult || !shift || lo > hi || lo < -128 || hi > 127) {
    bnh_fail("bnh_q8w_new: N %d K %d lo %d hi %d: expected N, K > 0, all four arrays and -128 <= lo <= hi <= 127", N, K,
             lo, hi);
    return nullptr;
  }
  for (int n = 0; n < N; n++)
    if (shift[n] < 0 || shift[n] > 31) {
      bnh_fail("bnh_q8w_new: shift[%d] = %d: expected a right shift in [0, 31]", n, shift[n]);
      return nullptr;
    }
  const int Nt = (int)bnh_round_up(N, RQ2_CH);  // every staging thread of a block owns one weight row
  const int Kt = (int)bnh_round_up(K, RQ4_BK);
  int8_t *hw = (int8_t *)calloc((size_t)Nt * Kt, 1);
  int32_t *hb = (int32_t *)calloc(Nt, 4), *hm = (int32_t *)calloc(Nt, 4), *hs = (int32_t *)calloc(Nt, 4);
  bnh_q8w *W = (bnh_q8w *)calloc(1, sizeof *W);
  if (!hw || !hb || !hm || !hs || !W) {
    free(hw); free(hb); free(hm); free(hs); free(W);
    bnh_fail("bnh_q8w_new: out of host memory");
    return nullptr;
  }
  for (int n = 0; n < N; n++) memcpy(hw + (size_t)n * Kt, w + (size_t)n * K, (size_t)K);
  for (int n = 0; n < N; n++) {
    uint32_t cs = 0;
    for (int k = 0; k < K; k++) cs += (uint32_t)(int32_t)w[(size_t)n * K + k];
    hb[n] = (int32_t)((uint32_t)bias[n] - (uint32_t)zx * cs);
    hm[n] = mult[n];
    hs[n] = shift[n];
  }
  W->N = N; W->K = K; W->Kt = Kt; W->Nt = Nt; W->zx = zx; W->zy = zy; W->lo = lo; W->hi = hi;
  W->all_s1 = 1;
  for (int n = 0; n < N; n++) W->all_s1 &= shift[n] >= 1;
  // the short epilogue clamps to [lo - zy, hi - zy] and adds zy bytewise: every clamped value must fit one byte
  W->fast = W->all_s1 && zy <= lo && lo <= hi && (long long)hi - zy <= 255;
  for (int n = 0; n < N; n++) W->fast &= llabs((long long)hb[n]) + (long long)K * 16384 < (1LL << 31);
  int32_t *hc = (int32_t *)calloc(2 * (size_t)Nt, 4), *he = (int32_t *)calloc(Nt, 4);
  if (!hc || !he) {
    free(hw); free(hb); free(hm); free(hs); free(hc); free(he); free(W);
    bnh_fail("bnh_q8w_new: out of host memory");
    return nullptr;
  }
  for (int n = 0; n < N && W->fast; n++) {
    const uint64_t c = (uint64_t)((int64_t)hb[n] * mult[n] + (1LL << 30) + (1LL << (30 + shift[n])));
    hc[n] = (int32_t)(uint32_t)c;
    hc[Nt + n] = (int32_t)(uint32_t)(c >> 32);
    he[n] = shift[n] - 1;
  }
  bool ok = (W->w = (int8_t *)bnh_malloc((size_t)Nt * Kt)) && (W->bias_eff = (int32_t *)bnh_malloc(4 * (size_t)Nt)) &&
            (W->mult = (int32_t *)bnh_malloc(4 * (size_t)Nt)) && (W->shift = (int32_t *)bnh_malloc(4 * (size_t)Nt)) &&
            !bnh_memcpy_h2d(W->w, hw, (size_t)Nt * Kt) && !bnh_memcpy_h2d(W->bias_eff, hb, 4 * (size_t)Nt) &&
            !bnh_memcpy_h2d(W->mult, hm, 4 * (size_t)Nt) && !bnh_memcpy_h2d(W->shift, hs, 4 * (size_t)Nt) &&
            (W->cq = (int32_t *)bnh_malloc(8 * (size_t)Nt)) && (W->e1 = (int32_t *)bnh_malloc(4 * (size_t)Nt)) &&
            !bnh_memcpy_h2d(W->cq, hc, 8 * (size_t)Nt) && !bnh_memcpy_h2d(W->e1, he, 4 * (size_t)Nt);
  free(hw); free(hb); free(hm); free(hs); free(hc); free(he);
  if (!ok) { bnh_q8w_free(W); return nullptr; }
  return W;
}

void bnh_q8w_free(bnh_q8w *W) {
  if (!W) return;
  if (W->w) (void)hipFree(W->w);
  if (W->bias_eff) (void)hipFree(W->bias_eff);
  if (W->mult) (void)hipFree(W->mult);
  if (W->shift) (void)hipFree(W->shift);
  if (W->cq) (void)hipFree(W->cq);
  if (W->e1) (void)hipFree(W->e1);
  free(W);
}

int bnh_gemm_s8_requant(const bnh_q8w *W, const int8_t *x, long long x_ws, int M, int B, int8_t *out,
                        long long out_ws, void *stream) {
  BNH_REQ(W && x && out && M > 0 && B > 0);
  BNH_REQ(M % 4 == 0 && ((uintptr_t)x & 3) == 0 && ((uintptr_t)out & 3) == 0);
  BNH_REQ(B == 1 || (x_ws % 4 == 0 && out_ws % 4 == 0 && x_ws >= (long long)W->K * M && out_ws >= (long long)W->N * M));
  BNH_REQ(W->K % 16 == 0);
  hipStream_t st = bnh_stream(stream);
  if (M % 16 == 0 && ((uintptr_t)x & 15) == 0 && (B == 1 || x_ws % 16 == 0) && W->Nt <= RQ4_MAXNT &&
      (long long)W->N * M < (1LL << 31)) {
    static int ncu = 0;
    if (!ncu) {
      int dev = 0;
      BNH_HIP(hipGetDevice(&dev));
      BNH_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
    }
    const int tpw = (int)bnh_ceil_div(M, RQ4_PIX), nblk = W->Nt / RQ4_CH;
    const long long nt = (long long)tpw * nblk * B;
    BNH_REQ(nt < (1LL << 31));
    const int grid = (int)(nt < ncu ? nt : ncu);
    // the ping-pong form stores 16 bytes per lane: 16-byte aligned output rows
    // BNH_RQ_FORM=pp / v4 selects an older form, for comparison
    static const char *form_env = getenv("BNH_RQ_FORM");
    static const int form = !form_env ? 6 : !strcmp(form_env, "v4") ? 4 : !strcmp(form_env, "pp") ? 5 : 6;
    if (form != 4 && ((uintptr_t)out & 15) == 0 && (B == 1 || out_ws % 16 == 0)) {
      if (form == 5)
        hipLaunchKernelGGL(W->all_s1 ? k_gemm_s8_requant_pp<true> : k_gemm_s8_requant_pp<false>, dim3(grid), dim3(512),
                           0, st, x, x_ws, M, W->K, W->Kt, tpw, nblk, (int)nt, W->w, W->bias_eff, W->mult, W->shift,
                           W->N, W->zy, W->lo, W->hi, out, out_ws);
      else {
        auto k = W->fast ? k_gemm_s8_requant_sr<2, 4, 4> : W->all_s1 ? k_gemm_s8_requant_sr<1, 4, 4>
                                                                     : k_gemm_s8_requant_sr<0, 4, 4>;
        hipLaunchKernelGGL(k, dim3(grid), dim3(512), 0, st, x, x_ws, M, W->K, W->Kt, tpw, nblk, (int)nt, W->w,
                           W->bias_eff, W->mult, W->shift, W->N, W->zy, W->lo, W->hi, out, out_ws, W->cq, W->e1);
      }
    } else
      hipLaunchKernelGGL(k_gemm_s8_requant4, dim3(grid), dim3(512), 0, st, x, x_ws, M, W->K, W->Kt, tpw, nblk, (int)nt,
                         W->w, W->bias_eff, W->mult, W->shift, W->N, W->zy, W->lo, W->hi, out, out_ws);
  } else {
    const int tpw = (int)bnh_ceil_div(M, RQ2_PIX);
    dim3 grid((unsigned)((long long)tpw * B), (unsigned)(W->Nt / RQ2_CH));
    hipLaunchKernelGGL(k_gemm_s8_requant2, grid, dim3(256), 0, st, x, x_ws, M, W->K, tpw, W->w, W->Kt, W->bias_eff,
                       W->mult, W->shift, W->N, W->zy, W->lo, W->hi, out, out_ws);
  }
  BNH_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
