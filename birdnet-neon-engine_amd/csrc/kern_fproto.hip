// The fp32 and fp16 prototype heads of libbnneon on gfx950: PROTO variant 0 (fp32 cells and prototypes,
// src/rt_ops_f32.c:548-570), PROTO_F32H (fp16-stored prototypes, fp32 arithmetic, src/rt_ops_f32.c:572-591) and
// PROTO variant 1 (fp16, src/rt_ops_f16.c:227-250). Each is the L2 normalisation of the cells (pc_l2norm_f32 /
// pc_l2norm_f16), the cells x prototypes product of which only the column maxima over a window's cells are kept
// (gemm_f32_colmax, pc_proto_colmax_f32h, gemm_f16_colmax), then the class logits (bnh_proto_logits, kern_proto.hip).
//
// Bit-identical to the reference. Every product sum is one fused multiply-add chain in the reference's order: fp32
// from +0 over k; fp16 from +0 over each K block (the fp16 GEMM's balanced blocks of at most 128 steps), the blocks'
// widened results summed in fp32 from +0. Matrix cores sum their products in an order of their own, so the chains
// run on the VALU: a thread owns 8 cells x 8 prototypes (64 fp32 chains, or 32 packed fp16 pairs), its operands two
// 16-byte LDS reads per k step each. The maximum over cells is exact and order-free (NaN-propagating FMAX).
//
// Prototypes are repacked at load into k-major rows [K][Npt] (Npt = Np rounded up to 256, zeros past Np): a block's
// 256 prototypes at one k are one contiguous 1 KB (fp32) or 512 B (fp16) run. A block is one window x 256
// prototypes, windows fastest, so the blocks in flight share their prototype tile in L2; it walks the window's cells
// 64 at a time.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "bnh_f16.h"
#include "bnh_internal.h"
#include "bnh_num.h"

struct bnh_fproto {
  int kind;     // 0 fp32 (PROTO variant 0), 1 fp16-stored / fp32 math (PROTO_F32H), 2 fp16 (PROTO variant 1)
  int Np, K, Npt;
  int nblk, bs;  // kind 2: the fp16 GEMM's K blocks
  void *w;       // k-major [K][Npt]: fp32 (kind 0) or fp16 bit patterns (kinds 1, 2)
};

// ------------------------------------------------------------------ L2 normalisation of the cells
// One wave per cell. The sum of squares is 8 fused chains (channel c feeds chain c % 8, in order of c: the two
// 4-lane accumulators of 8-channel steps), combined as ((t0 + t1) + (t2 + t3)) with t_j = chain_j + chain_{j+4};
// lanes 0..7 run the chains over a 512-float LDS chunk the whole wave stages. den = sqrtf(sum) + eps, a = x / den
// (correctly rounded division); F16: fp16 cells widened, a rounded to fp16 (nearest even).
#define L2_CHUNK 512
template <bool F16>
__global__ __launch_bounds__(256) void k_l2norm(const void *__restrict__ xv, long long x_ws, int P, int C, int ld,
                                                float eps, void *__restrict__ av, long long a_ws, long long cells) {
  __shared__ float stage[4][L2_CHUNK];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const long long cell = (long long)blockIdx.x * 4 + wv;
  const bool live = cell < cells;
  const int w = live ? (int)(cell / P) : 0, p = live ? (int)(cell % P) : 0;
  const float *r = F16 ? nullptr : (const float *)xv + w * x_ws + (long long)p * ld;
  const h16 *rh = F16 ? (const h16 *)xv + w * x_ws + (long long)p * ld : nullptr;
  float chain = 0.f;
  for (int c0 = 0; c0 < C; c0 += L2_CHUNK) {
    const int n = C - c0 < L2_CHUNK ? C - c0 : L2_CHUNK;
    if (live)
      for (int i = lane; i < n; i += 64) stage[wv][i] = F16 ? (float)rh[c0 + i] : r[c0 + i];
    __syncthreads();
    if (live && lane < 8)
      for (int i = lane; i < n; i += 8) chain = __builtin_fmaf(stage[wv][i], stage[wv][i], chain);
    __syncthreads();
  }
  if (!live) return;
  const float s1 = __shfl(chain, (lane & 3) + 4);
  const float t = chain + s1;  // t_j in lanes 0..3
  const float t0 = __shfl(t, 0), t1 = __shfl(t, 1), t2 = __shfl(t, 2), t3 = __shfl(t, 3);
  const float den = __builtin_sqrtf((t0 + t1) + (t2 + t3)) + eps;
  if (F16) {
    h16 *a = (h16 *)av + w * a_ws + (long long)p * C;
    for (int c = lane; c < C; c += 64) a[c] = f2h((float)rh[c] / den);
  } else {
    float *a = (float *)av + w * a_ws + (long long)p * C;
    for (int c = lane; c < C; c += 64) a[c] = r[c] / den;
  }
}

// ------------------------------------------------------------------ fp32 column maxima (kinds 0 and 1)
#define FP_BM 64   // cells per tile
#define FP_BN 256  // prototypes per block
#define FP_KC 16   // k steps per LDS stage
#define FP_AS 68   // As row stride in floats ([k][cell]; 16-byte aligned rows)
// WH: prototypes stored as fp16, widened exactly as they are staged (PROTO_F32H)
template <bool WH>
__global__ __launch_bounds__(256) void k_colmax_f32(const float *__restrict__ a, long long a_ws, int P, int K,
                                                    const void *__restrict__ wv, int Npt, int Np,
                                                    float *__restrict__ colmax, long long cm_ws, int B) {
  __shared__ __attribute__((aligned(16))) float As[2][FP_KC][FP_AS];
  __shared__ __attribute__((aligned(16))) float Ws[2][FP_KC][FP_BN];
  const int tid = threadIdx.x, cg = tid & 7, pg = tid >> 3;
  const int win = (int)(blockIdx.x % (unsigned)B), n0 = (int)(blockIdx.x / (unsigned)B) * FP_BN;
  const float *aw = a + win * a_ws;
  // loader roles: A, cell tid / 4 and k 4 (tid % 4) .. + 3; W fp32, rows (tid + 256 j) / 64, 4 prototypes each;
  // W fp16, rows (tid + 256 j) / 32, 8 prototypes each
  const int la_c = tid >> 2, la_k = 4 * (tid & 3);
  float4 ra;
  float4 rw[WH ? 1 : 4];
  uint4 rh[WH ? 2 : 1];
  float mx[8];
#pragma unroll
  for (int j = 0; j < 8; j++) mx[j] = -INFINITY;
  for (int m0 = 0; m0 < P; m0 += FP_BM) {
    const int crow = m0 + la_c < P ? m0 + la_c : P - 1;  // rows past P repeat the last cell; their sums are unused
    const float *arow = aw + (long long)crow * K;
    auto load = [&](int k0) {
      ra = k0 + la_k < K ? *(const float4 *)(arow + k0 + la_k) : make_float4(0.f, 0.f, 0.f, 0.f);
      if (WH) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
          const int i = tid + 256 * j, row = i >> 5, c8 = i & 31;
          rh[j] = k0 + row < K ? *(const uint4 *)((const uint16_t *)wv + (long long)(k0 + row) * Npt + n0 + 8 * c8)
                               : make_uint4(0, 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int i = tid + 256 * j, row = i >> 6, c4 = i & 63;
          rw[j] = k0 + row < K ? *(const float4 *)((const float *)wv + (long long)(k0 + row) * Npt + n0 + 4 * c4)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    };
    auto store = [&](int buf) {
      As[buf][la_k + 0][la_c] = ra.x;
      As[buf][la_k + 1][la_c] = ra.y;
      As[buf][la_k + 2][la_c] = ra.z;
      As[buf][la_k + 3][la_c] = ra.w;
      if (WH) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
          const int i = tid + 256 * j, row = i >> 5, c8 = i & 31;
          const h2 v[4] = {__builtin_bit_cast(h2, rh[j].x), __builtin_bit_cast(h2, rh[j].y),
                           __builtin_bit_cast(h2, rh[j].z), __builtin_bit_cast(h2, rh[j].w)};
          *(float4 *)&Ws[buf][row][8 * c8] = make_float4((float)v[0].x, (float)v[0].y, (float)v[1].x, (float)v[1].y);
          *(float4 *)&Ws[buf][row][8 * c8 + 4] = make_float4((float)v[2].x, (float)v[2].y, (float)v[3].x, (float)v[3].y);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int i = tid + 256 * j, row = i >> 6, c4 = i & 63;
          *(float4 *)&Ws[buf][row][4 * c4] = rw[j];
        }
      }
    };
    float acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int j = 0; j < 8; j++) acc[i][j] = 0.f;
    __syncthreads();  // the previous tile's last reads of buffer 0 are done
    load(0);
    store(0);
    __syncthreads();
    for (int k0 = 0, cur = 0; k0 < K; k0 += FP_KC, cur ^= 1) {
      const bool more = k0 + FP_KC < K;
      if (more) load(k0 + FP_KC);
      const int kn = K - k0 < FP_KC ? K - k0 : FP_KC;  // 16 or 8 (K % 8 == 0)
      for (int kk = 0; kk < kn; kk += 8) {
#pragma unroll
        for (int k = kk; k < kk + 8; k++) {
          const float4 a0 = *(const float4 *)&As[cur][k][8 * cg], a1 = *(const float4 *)&As[cur][k][8 * cg + 4];
          const float4 w0 = *(const float4 *)&Ws[cur][k][8 * pg], w1 = *(const float4 *)&Ws[cur][k][8 * pg + 4];
          const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
          const float wt[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
          for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < 8; j++) acc[i][j] = __builtin_fmaf(wt[j], av[i], acc[i][j]);
        }
      }
      if (more) store(cur ^ 1);
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (m0 + 8 * cg + i < P)
#pragma unroll
        for (int j = 0; j < 8; j++) mx[j] = bnh_fmax(mx[j], acc[i][j]);
  }
  // the 8 cell groups of a prototype group are lanes l ^ 1, 2, 4
#pragma unroll
  for (int j = 0; j < 8; j++) {
    mx[j] = bnh_fmax(mx[j], __shfl_xor(mx[j], 1));
    mx[j] = bnh_fmax(mx[j], __shfl_xor(mx[j], 2));
    mx[j] = bnh_fmax(mx[j], __shfl_xor(mx[j], 4));
  }
  float v = mx[0];
#pragma unroll
  for (int j = 1; j < 8; j++)
    if (cg == j) v = mx[j];
  const int n = n0 + 8 * pg + cg;
  if (n < Np) colmax[win * cm_ws + n] = v;
}

// ------------------------------------------------------------------ fp16 column maxima (kind 2)
#define HP_KC 32  // k steps per LDS stage
#define HP_AS 72  // As row stride in halves ([k][cell]; 16-byte aligned rows)
__global__ __launch_bounds__(256) void k_colmax_f16(const uint16_t *__restrict__ a, long long a_ws, int P, int K,
                                                    const uint16_t *__restrict__ w, int Npt, int Np, int bs, int nblk,
                                                    float *__restrict__ colmax, long long cm_ws, int B) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][HP_KC][HP_AS];
  __shared__ __attribute__((aligned(16))) uint4 Ws[2][HP_KC][FP_BN / 8];
  const int tid = threadIdx.x, cg = tid & 7, pg = tid >> 3;
  const int win = (int)(blockIdx.x % (unsigned)B), n0 = (int)(blockIdx.x / (unsigned)B) * FP_BN;
  const uint16_t *aw = a + win * a_ws;
  // loader roles: A, cell tid / 4 and k 8 (tid % 4) .. + 7; W rows (tid + 256 j) / 32, 8 prototypes each
  const int la_c = tid >> 2, la_k = 8 * (tid & 3);
  uint4 ra, rw[4];
  float mx[8];
#pragma unroll
  for (int j = 0; j < 8; j++) mx[j] = -INFINITY;
  for (int m0 = 0; m0 < P; m0 += FP_BM) {
    const int crow = m0 + la_c < P ? m0 + la_c : P - 1;
    const uint16_t *arow = aw + (long long)crow * K;
    auto load = [&](int k0) {
      ra = k0 + la_k < K ? *(const uint4 *)(arow + k0 + la_k) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int i = tid + 256 * j, row = i >> 5, c8 = i & 31;
        rw[j] = k0 + row < K ? *(const uint4 *)(w + (long long)(k0 + row) * Npt + n0 + 8 * c8) : make_uint4(0, 0, 0, 0);
      }
    };
    auto store = [&](int buf) {
      const uint32_t v[4] = {ra.x, ra.y, ra.z, ra.w};
#pragma unroll
      for (int u = 0; u < 4; u++) {
        As[buf][la_k + 2 * u][la_c] = (uint16_t)(v[u] & 0xffffu);
        As[buf][la_k + 2 * u + 1][la_c] = (uint16_t)(v[u] >> 16);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int i = tid + 256 * j, row = i >> 5, c8 = i & 31;
        Ws[buf][row][c8] = rw[j];
      }
    };
    h2 acc[8][4];
    float fb[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
#pragma unroll
      for (int q = 0; q < 4; q++) acc[i][q] = (h2){(h16)0.0f, (h16)0.0f};
#pragma unroll
      for (int j = 0; j < 8; j++) fb[i][j] = 0.f;
    }
    __syncthreads();
    load(0);
    store(0);
    __syncthreads();
    int kend = bs < K ? bs : K;  // the end of the current K block
    for (int k0 = 0, cur = 0; k0 < K; k0 += HP_KC, cur ^= 1) {
      const bool more = k0 + HP_KC < K;
      if (more) load(k0 + HP_KC);
      const int kn = K - k0 < HP_KC ? K - k0 : HP_KC;  // a multiple of 8
      for (int kk = 0; kk < kn; kk += 8) {
#pragma unroll
        for (int k = kk; k < kk + 8; k++) {
          const uint4 av4 = *(const uint4 *)&As[cur][k][8 * cg];
          const uint4 wv4 = Ws[cur][k][pg];
          const h2 ap[4] = {__builtin_bit_cast(h2, av4.x), __builtin_bit_cast(h2, av4.y), __builtin_bit_cast(h2, av4.z),
                            __builtin_bit_cast(h2, av4.w)};
          const h2 wp[4] = {__builtin_bit_cast(h2, wv4.x), __builtin_bit_cast(h2, wv4.y), __builtin_bit_cast(h2, wv4.z),
                            __builtin_bit_cast(h2, wv4.w)};
#pragma unroll
          for (int i = 0; i < 8; i++) {
            const h16 ai = (i & 1) ? ap[i >> 1].y : ap[i >> 1].x;
            const h2 as = (h2){ai, ai};
#pragma unroll
            for (int q = 0; q < 4; q++) acc[i][q] = __builtin_elementwise_fma(wp[q], as, acc[i][q]);
          }
        }
        if (k0 + kk + 8 == kend) {  // a K block ends
          if (nblk > 1) {
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
              for (int q = 0; q < 4; q++) {
                fb[i][2 * q] = fb[i][2 * q] + (float)acc[i][q].x;
                fb[i][2 * q + 1] = fb[i][2 * q + 1] + (float)acc[i][q].y;
                acc[i][q] = (h2){(h16)0.0f, (h16)0.0f};
              }
          }
          kend = kend + bs < K ? kend + bs : K;
        }
      }
      if (more) store(cur ^ 1);
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (m0 + 8 * cg + i < P)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float lo = nblk > 1 ? fb[i][2 * q] : (float)acc[i][q].x;
          const float hi = nblk > 1 ? fb[i][2 * q + 1] : (float)acc[i][q].y;
          mx[2 * q] = bnh_fmax(mx[2 * q], lo);
          mx[2 * q + 1] = bnh_fmax(mx[2 * q + 1], hi);
        }
  }
#pragma unroll
  for (int j = 0; j < 8; j++) {
    mx[j] = bnh_fmax(mx[j], __shfl_xor(mx[j], 1));
    mx[j] = bnh_fmax(mx[j], __shfl_xor(mx[j], 2));
    mx[j] = bnh_fmax(mx[j], __shfl_xor(mx[j], 4));
  }
  float v = mx[0];
#pragma unroll
  for (int j = 1; j < 8; j++)
    if (cg == j) v = mx[j];
  const int n = n0 + 8 * pg + cg;
  if (n < Np) colmax[win * cm_ws + n] = v;
}

// ================================================================== host side
extern "C" {

bnh_fproto *bnh_fproto_new(int kind, int Np, int K, const void *w) {
  if (kind < 0 || kind > 2 || Np <= 0 || Np % 8 || K <= 0 || K % 8 || K > (1 << 20) || !w) {
    bnh_fail("bnh_fproto_new: kind %d Np %d K %d: expected kind 0..2, Np and K positive multiples of 8, K <= 2^20 and "
             "the prototype tensor", kind, Np, K);
    return nullptr;
  }
  const int Npt = (int)bnh_round_up(Np, FP_BN);
  const size_t esz = kind == 0 ? 4 : 2, bytes = (size_t)K * Npt * esz;
  void *h = calloc(bytes, 1);
  bnh_fproto *W = (bnh_fproto *)calloc(1, sizeof *W);
  if (!h || !W) {
    free(h); free(W);
    bnh_fail("bnh_fproto_new: out of host memory");
    return nullptr;
  }
  const int n16 = Np / 16;
  for (int n = 0; n < Np; n++) {
    // the package panel holding prototype n and its column in the panel
    size_t base, step;
    if (kind < 2) {
      base = (size_t)(n / 8) * K * 8 + n % 8;  // [Np/8][K][8]
      step = 8;
    } else if (n / 16 < n16) {
      base = (size_t)(n / 16) * K * 16 + n % 16;  // [Np/16][K][16]
      step = 16;
    } else {
      base = (size_t)n16 * K * 16 + (n - 16 * n16);  // the tail panel [K][8]
      step = 8;
    }
    for (int k = 0; k < K; k++) {
      const size_t src = base + (size_t)k * step, dst = (size_t)k * Npt + n;
      if (esz == 4) ((float *)h)[dst] = ((const float *)w)[src];
      else ((uint16_t *)h)[dst] = ((const uint16_t *)w)[src];
    }
  }
  W->kind = kind; W->Np = Np; W->K = K; W->Npt = Npt;
  W->nblk = (K + 127) / 128;
  W->bs = ((K + W->nblk - 1) / W->nblk + 7) & ~7;
  const bool ok = (W->w = bnh_malloc(bytes)) && !bnh_memcpy_h2d(W->w, h, bytes);
  free(h);
  if (!ok) { bnh_fproto_free(W); return nullptr; }
  return W;
}

void bnh_fproto_free(bnh_fproto *W) {
  if (!W) return;
  if (W->w) (void)hipFree(W->w);
  free(W);
}

int bnh_l2norm_cells(const void *x, long long x_ws, int P, int C, int ld, float eps, int f16, void *a, long long a_ws,
                     int B, void *stream) {
  BNH_REQ(x && a && P > 0 && C > 0 && B > 0);
  BNH_REQ(C % 8 == 0 && ld >= C);
  BNH_REQ(B == 1 || (x_ws >= (long long)(P - 1) * ld + C && a_ws >= (long long)P * C));
  const long long cells = (long long)P * B;
  if (f16)
    hipLaunchKernelGGL(k_l2norm<true>, dim3((unsigned)bnh_ceil_div(cells, 4)), dim3(256), 0, bnh_stream(stream), x, x_ws,
                       P, C, ld, eps, a, a_ws, cells);
  else
    hipLaunchKernelGGL(k_l2norm<false>, dim3((unsigned)bnh_ceil_div(cells, 4)), dim3(256), 0, bnh_stream(stream), x,
                       x_ws, P, C, ld, eps, a, a_ws, cells);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_fproto_colmax(const void *a, long long a_ws, int P, const bnh_fproto *W, float *colmax, long long cm_ws, int B,
                      void *stream) {
  BNH_REQ(a && W && colmax && P > 0 && B > 0);
  BNH_REQ(((uintptr_t)a & 15) == 0 && (B == 1 || a_ws % 8 == 0));
  BNH_REQ(B == 1 || (a_ws >= (long long)P * W->K && cm_ws >= W->Np));
  const long long blocks = (long long)B * (W->Npt / FP_BN);
  BNH_REQ(blocks < (1LL << 31));
  if (B == 1) a_ws = cm_ws = 0;
  if (W->kind == 2)
    hipLaunchKernelGGL(k_colmax_f16, dim3((unsigned)blocks), dim3(256), 0, bnh_stream(stream), (const uint16_t *)a, a_ws,
                       P, W->K, (const uint16_t *)W->w, W->Npt, W->Np, W->bs, W->nblk, colmax, cm_ws, B);
  else if (W->kind == 1)
    hipLaunchKernelGGL(k_colmax_f32<true>, dim3((unsigned)blocks), dim3(256), 0, bnh_stream(stream), (const float *)a,
                       a_ws, P, W->K, (const void *)W->w, W->Npt, W->Np, colmax, cm_ws, B);
  else
    hipLaunchKernelGGL(k_colmax_f32<false>, dim3((unsigned)blocks), dim3(256), 0, bnh_stream(stream), (const float *)a,
                       a_ws, P, W->K, (const void *)W->w, W->Npt, W->Np, colmax, cm_ws, B);
  BNH_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
