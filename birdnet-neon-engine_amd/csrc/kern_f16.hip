// fp16 pointwise-convolution GEMM (libbnneon's gemm_f16, src/gemm_f16.c, the PW op of the fp16 family) on gfx950,
// in two forms:
//  - k_gemm_f16e (bnh_gemm_f16): the reference's own arithmetic, bit-identical: per output an fp16 FMA chain over
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
  uint16_t *w;    // [Nt][Kp] (the MFMA form)
  uint16_t *wk;   // [Kp][Nt] (the exact form)
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

// 4 waves as 2 (rows) x 2 (channels); a wave computes 32 rows x 64 channels (2 x 4 MFMA tiles). Each block resolves
// its 64 rows' window, A / output / residual / gate addresses into LDS once. GATE: A's columns are multiplied by the
// window's fp16 gates as they are loaded (the fp16 SE's scaling, one fp16 rounding per product, as in k_gemm_f16e).
// VEC: each wave's 16 x 64 tile leaves the accumulators through LDS (bias, rounding and activation done in the
// accumulator layout), and goes out as 16-byte rows of 8 channels with their residual added in fp16.
template <bool GATE, bool VEC>
__global__ __launch_bounds__(256) void k_gemm_f16(const uint16_t *__restrict__ A, long long a_ws, int lda, int M,
                                                  double rM, long long rows, const uint16_t *__restrict__ wt,
                                                  const float *__restrict__ bias, int Kp, int Np, Epi16Dev e,
                                                  const uint16_t *__restrict__ gh, long long gh_ws) {
  constexpr int TS = 72;  // the tile's LDS row stride in halves (64 channels + 8)
  __shared__ long long s_a[64], s_o[64], s_r[64], s_g[GATE ? 64 : 1];
  __shared__ __attribute__((aligned(16))) uint16_t s_t[VEC ? 4 : 1][VEC ? 16 * TS : 1];
  __shared__ uint32_t s_t01[16];  // the SiLU table in LDS (c0 | c1 << 16, c2) for the packed form
  __shared__ uint16_t s_t2[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // the channel blocks of a row block are consecutive logical blocks on one XCD: its output rows' cache lines fill
  // in that XCD's L2 while the row block is being written (partial lines from far-apart blocks cost HBM write rate)
  const int nnb = (Np + 127) / 128;
  const unsigned lb = bnh_xcd_block(blockIdx.x, gridDim.x);
  const long long rowB = (long long)(lb / nnb) * 64;
  const int nblk = (int)(lb % nnb);
  if (threadIdx.x < 64) {
    const long long r = rowB + threadIdx.x < rows ? rowB + threadIdx.x : rows - 1;  // a valid row past the end
    const int w = bnh_div(r, M, rM), m = (int)(r - (long long)w * M);
    s_a[threadIdx.x] = w * a_ws + (long long)m * lda;
    long long orow = m;
    if (e.opad) {
      const int y = m / e.ow;
      orow = (long long)(y + e.opad) * (e.ow + 2 * e.opad) + (m - y * e.ow) + e.opad;
    }
    s_o[threadIdx.x] = w * e.out_ws + orow * e.ldo;
    s_r[threadIdx.x] = e.res ? w * e.res_ws + (long long)m * e.ldr : 0;
    if (GATE) s_g[threadIdx.x] = w * gh_ws;
  }
  if (threadIdx.x < 16) {
    s_t01[threadIdx.x] = (uint32_t)k_silu_c0[threadIdx.x] | ((uint32_t)k_silu_c1[threadIdx.x] << 16);
    s_t2[threadIdx.x] = k_silu_c2[threadIdx.x];
  }
  __syncthreads();
  const int lr0 = wm * 32, n0 = nblk * 128 + wn * 64;
  if (rowB + lr0 >= rows) return;
  const int kc = (lane >> 4) * 8;  // this lane's k chunk within a 32-wide step (halves)
  const uint16_t *ap[2], *gp[2];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    ap[t] = A + s_a[lr0 + 16 * t + (lane & 15)] + kc;
    gp[t] = GATE ? gh + s_g[lr0 + 16 * t + (lane & 15)] + kc : nullptr;
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
    for (int t = 0; t < 2; t++) {
      a[t] = in ? *(const v8h *)(ap[t] + k) : (v8h){};
      if (GATE && in) a[t] = a[t] * *(const v8h *)(gp[t] + k);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) b[j] = in ? *(const v8h *)(bp + (long long)16 * j * Kp + k) : (v8h){};
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], b[j], acc[t][j], 0, 0, 0);
  }
  // accumulator lane layout: acc[t][j][r] = row 16 t + 4 (lane >> 4) + r, channel 16 j + (lane & 15)
  float bn[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int n = n0 + 16 * j + (lane & 15);
    bn[j] = n < Np ? bias[n] : 0.f;
  }
  const int nlim = Np < e.ldo ? Np : e.ldo;  // channels stored
#pragma unroll
  for (int t = 0; t < 2; t++) {
    if (VEC) {
      uint16_t *T = s_t[wave];
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          // fp32 adds, then one rounding each to fp16 (nearest even); the SiLU on the pair in packed fp16
          h2 v = (h2){f2h(acc[t][j][r] + bn[j]), f2h(acc[t][j][r + 1] + bn[j])};
          if (e.act == 1) v = silu2_lut(v, s_t01, s_t2);
          else if (e.act == 2) v = (h2){hmax(v[0], (h16)0.0f), hmax(v[1], (h16)0.0f)};
          T[(4 * (lane >> 4) + r) * TS + 16 * j + (lane & 15)] = hbits(v[0]);
          T[(4 * (lane >> 4) + r + 1) * TS + 16 * j + (lane & 15)] = hbits(v[1]);
        }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // 16 rows x 8 chunks of 8 channels: two chunks per lane
      const int ch = lane & 7;
      const int n = n0 + 8 * ch;
      v8h rv[2];
#pragma unroll
      for (int it = 0; it < 2; it++) {  // the residual chunks first (out and res may alias)
        const int rr = 2 * (lane >> 3) + it, lr = lr0 + 16 * t + rr;
        rv[it] = e.res && n < nlim && rowB + lr < rows ? *(const v8h *)(e.res + s_r[lr] + n) : (v8h){};
      }
#pragma unroll
      for (int it = 0; it < 2; it++) {
        const int rr = 2 * (lane >> 3) + it, lr = lr0 + 16 * t + rr;
        if (n < nlim && rowB + lr < rows) {
          v8h y = *(const v8h *)(T + rr * TS + 8 * ch);
          if (e.res) y = y + rv[it];
          *(v8h *)(e.out + s_o[lr] + n) = y;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int n = n0 + 16 * j + (lane & 15);
        if (n >= nlim) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int lr = lr0 + 16 * t + 4 * (lane >> 4) + r;
          if (rowB + lr >= rows) continue;
          h16 v = f2h(acc[t][j][r] + bn[j]);
          if (e.act == 1) v = silu_lut_h(v);
          else if (e.act == 2) v = hmax(v, (h16)0.0f);
          if (e.res) v = v + hfrom(e.res[s_r[lr] + n]);
          e.out[s_o[lr] + n] = hbits(v);
        }
      }
    }
  }
}

// The same GEMM with the reference's own arithmetic (src/gemm_f16.c:49-171), so the outputs are bit-identical: per
// output an fp16 FMA chain over each K block (kblocks: ceil(Kp / 128) blocks, balanced, multiples of 8) from +0,
// the block results summed in fp32 when there are several (then + the fp32 bias, one rounding), else + the fp16
// bias in fp16; then the epilogue above. No MFMA (its accumulation is fp32): packed fp16 FMAs on the VALU, each
// lane one IEEE fp16 fused multiply-add, two channels per instruction.
// A block owns TN = 8 TC channels (TC = 4..16 thread columns, chosen per layer so the channel tiles cover Np with
// the least padding) x BM = 4 TR rows (TR = min(256 / TC, 64) thread rows; threads past TC x TR only load); a thread
// computes 4 rows x 8 channels (16 packed accumulators). K goes through LDS 32 steps at a time: A as it lies
// ([row][k], a row stride of 17 dwords so the 4-row reads of a wave hit distinct banks), W from its k-major copy
// ([k][channel], a thread's 8 channels one 16-byte read). The next chunk's global loads are issued before the
// current chunk is computed. Epilogue: the SiLU two channels at a time in packed fp16 with its table in LDS, 16-byte
// residual loads and stores (VEC).
#define FE_KC 32
#define FE_AS 17   // A row stride in dwords (34 halves)
#define FE_BM 256  // rows per block at most

// GATE: A's columns are multiplied by the window's fp16 gates gh [K] as they are staged (the fp16 SE's in-place
// scaling of A, src/rt_ops_f32.c:256-327, done in the A-load: the same fp16 products, no pass over A)
// MB: the fp32 sums of several K blocks (false when the launch has one K block, or one K block per block: the 32
// registers of those sums then stay free, 4 -> 5 waves per SIMD)
template <bool VEC, bool RES, bool GATE, bool MB>
__global__ __launch_bounds__(256) void k_gemm_f16e(const uint16_t *__restrict__ A, long long a_ws, int lda, int M,
                                                   double rM, long long rows, const uint16_t *__restrict__ wk, int Ntp,
                                                   const float *__restrict__ b32, const uint16_t *__restrict__ b16,
                                                   int Kp, int Np, int bs, int TC, Epi16Dev e,
                                                   const uint16_t *__restrict__ gh, long long gh_ws,
                                                   uint16_t *__restrict__ part, int nsplit) {
  const int TR = 256 / TC < 64 ? 256 / TC : 64, BM = 4 * TR, TN = 8 * TC;
  __shared__ __attribute__((aligned(16))) uint32_t As[FE_BM * FE_AS];
  __shared__ __attribute__((aligned(16))) uint4 Ws[FE_KC * 16];
  __shared__ long long s_a[FE_BM], s_o[FE_BM], s_r[FE_BM], s_g[GATE ? FE_BM : 1];
  __shared__ uint32_t s_t01[16];
  __shared__ uint16_t s_t2[16];
  const int tid = threadIdx.x, tc = tid % TC, tr = tid / TC;
  const bool active = tr < TR;
  // 1-D grid of (row block, channel tile) pairs, channel tile fastest, after the XCD remap: the blocks that write the
  // parts of the same output rows run together under one L2, which merges their partial cache lines
  // part: one K block per block (si, fastest), its fp16 chain results into part [si][rows][Np] for the combining kernel
  const int nct = (Np + TN - 1) / TN;
  const unsigned lb0 = bnh_xcd_block(blockIdx.x, gridDim.x), si = part ? lb0 % nsplit : 0;
  const unsigned lb = part ? lb0 / nsplit : lb0;
  const long long rowB = (long long)(lb / nct) * BM;
  const int n0 = (int)(lb % nct) * TN;
  const int kbeg = (int)si * bs, Kend = part ? (kbeg + bs < Kp ? kbeg + bs : Kp) : Kp;
  for (int i = tid; i < BM; i += 256) {
    const long long row = rowB + i < rows ? rowB + i : rows - 1;
    const int w = bnh_div(row, M, rM), m = (int)(row - (long long)w * M);
    s_a[i] = w * a_ws + (long long)m * lda;
    long long orow = m;
    if (e.opad) {
      const int y = m / e.ow;
      orow = (long long)(y + e.opad) * (e.ow + 2 * e.opad) + (m - y * e.ow) + e.opad;
    }
    s_o[i] = w * e.out_ws + orow * e.ldo;
    s_r[i] = w * e.res_ws + (long long)m * e.ldr;
    if (GATE) s_g[i] = w * gh_ws;
  }
  if (tid < 16) {
    s_t01[tid] = (uint32_t)k_silu_c0[tid] | ((uint32_t)k_silu_c1[tid] << 16);
    s_t2[tid] = k_silu_c2[tid];
  }
  __syncthreads();
  // chunk loader: A rows [BM][kn] and W rows [kn][TN] of k0 into registers (kn a multiple of 8)
  uint4 ra[FE_BM * FE_KC / 8 / 256], rw[2], rg[GATE ? FE_BM * FE_KC / 8 / 256 : 1];
  const int nav = BM * (FE_KC / 8), nwv = FE_KC * TC;
  auto load = [&](int k0, int kn) {
#pragma unroll
    for (int j = 0; j < FE_BM * FE_KC / 8 / 256; j++) {
      const int i = tid + 256 * j, r = i / (FE_KC / 8), kc = (i % (FE_KC / 8)) * 8;
      ra[j] = i < nav && kc < kn ? *(const uint4 *)(A + s_a[r] + k0 + kc) : make_uint4(0, 0, 0, 0);
      if (GATE) rg[j] = i < nav && kc < kn ? *(const uint4 *)(gh + s_g[r] + k0 + kc) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int i = tid + 256 * j, k = i / TC, c = i - k * TC;
      rw[j] = i < nwv && k < kn ? *(const uint4 *)(wk + (long long)(k0 + k) * Ntp + n0 + 8 * c)
                                : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int j = 0; j < FE_BM * FE_KC / 8 / 256; j++) {
      const int i = tid + 256 * j, r = i / (FE_KC / 8), kc = (i % (FE_KC / 8)) * 8;
      if (i < nav) {
        uint32_t *d = As + r * FE_AS + kc / 2;
        if (GATE) {  // a x gate, two columns at a time (IEEE fp16 products)
          const uint32_t av[4] = {ra[j].x, ra[j].y, ra[j].z, ra[j].w}, gv[4] = {rg[j].x, rg[j].y, rg[j].z, rg[j].w};
#pragma unroll
          for (int u = 0; u < 4; u++)
            d[u] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, av[u]) * __builtin_bit_cast(h2, gv[u]));
        } else {
          d[0] = ra[j].x; d[1] = ra[j].y; d[2] = ra[j].z; d[3] = ra[j].w;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int i = tid + 256 * j;
      if (i < nwv) Ws[i] = rw[j];
    }
  };
  h2 acc[4][4];
  float fb[MB ? 4 : 1][MB ? 8 : 1];
#pragma unroll
  for (int r = 0; r < 4; r++)
#pragma unroll
    for (int p = 0; p < 4; p++) acc[r][p] = (h2){(h16)0.0f, (h16)0.0f};
  if constexpr (MB) {
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int c = 0; c < 8; c++) fb[r][c] = 0.f;
  }
  const int nblk = (Kp + bs - 1) / bs;
  int kb = kbeg, k0 = kbeg;
  int kn = bs < FE_KC ? bs : FE_KC;
  if (kn > Kend - kbeg) kn = Kend - kbeg;
  load(kbeg, kn);
  const uint32_t *Ar = As + 4 * (active ? tr : 0) * FE_AS;
  const uint4 *Wt = Ws + tc;
  while (true) {
    __syncthreads();  // the previous chunk's reads are done
    store();
    __syncthreads();
    // the next chunk: within this K block, or the first of the next
    const int ke = kb + bs < Kend ? kb + bs : Kend;
    int nk0 = k0 + kn, nkb = kb;
    if (nk0 >= ke) nkb = nk0 = ke;
    const int nke = nkb + bs < Kend ? nkb + bs : Kend;
    const int nkn = nk0 < Kend ? (nke - nk0 < FE_KC ? nke - nk0 : FE_KC) : 0;
    if (nkn) load(nk0, nkn);
    if (active) {
      for (int k = 0; k < kn; k += 2) {
        uint32_t a[4];
#pragma unroll
        for (int r = 0; r < 4; r++) a[r] = Ar[r * FE_AS + k / 2];
        const uint4 w0 = Wt[k * TC], w1 = Wt[(k + 1) * TC];
        const h2 wa[4] = {__builtin_bit_cast(h2, w0.x), __builtin_bit_cast(h2, w0.y), __builtin_bit_cast(h2, w0.z),
                          __builtin_bit_cast(h2, w0.w)};
        const h2 wb[4] = {__builtin_bit_cast(h2, w1.x), __builtin_bit_cast(h2, w1.y), __builtin_bit_cast(h2, w1.z),
                          __builtin_bit_cast(h2, w1.w)};
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const h2 av = __builtin_bit_cast(h2, a[r]);
          const h2 lo = (h2){av.x, av.x}, hi = (h2){av.y, av.y};
#pragma unroll
          for (int p = 0; p < 4; p++) acc[r][p] = __builtin_elementwise_fma(wa[p], lo, acc[r][p]);
#pragma unroll
          for (int p = 0; p < 4; p++) acc[r][p] = __builtin_elementwise_fma(wb[p], hi, acc[r][p]);
        }
      }
      if constexpr (MB) {
        if (k0 + kn >= ke && nblk > 1 && !part) {  // a K block ends: its fp16 results into the fp32 sums
#pragma unroll
          for (int r = 0; r < 4; r++)
#pragma unroll
            for (int p = 0; p < 4; p++) {
              fb[r][2 * p] = fb[r][2 * p] + (float)acc[r][p].x;
              fb[r][2 * p + 1] = fb[r][2 * p + 1] + (float)acc[r][p].y;
              acc[r][p] = (h2){(h16)0.0f, (h16)0.0f};
            }
        }
      }
    }
    if (!nkn) break;
    kb = nkb; k0 = nk0; kn = nkn;
  }
  // epilogue
  const int n = n0 + 8 * tc;
  if (part) {  // the block's fp16 results (Np % 8 == 0: a thread's 8 channels are all below Np or all past it)
    if (!active || n >= Np) return;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const long long row = rowB + 4 * tr + r;
      if (row >= rows) break;
      *(uint4 *)(part + ((long long)si * rows + row) * Np + n) =
          make_uint4(__builtin_bit_cast(uint32_t, acc[r][0]), __builtin_bit_cast(uint32_t, acc[r][1]),
                     __builtin_bit_cast(uint32_t, acc[r][2]), __builtin_bit_cast(uint32_t, acc[r][3]));
    }
    return;
  }
  const int nend = Np < e.ldo ? Np : e.ldo;
  if (!active || n >= nend) return;
  const bool full = VEC && n + 8 <= nend;
  float bias32[8];
  uint16_t bias16[8];
#pragma unroll
  for (int c = 0; c < 8; c++) {
    bias32[c] = n + c < nend ? b32[n + c] : 0.f;
    bias16[c] = n + c < nend ? b16[n + c] : 0;
  }
  // RES (with VEC): the residuals of the thread's 4 rows loaded together before any store (which the compiler may not
  // move them past: out and res could alias)
  uint4 rvs[4];
  if (RES && full) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int lr = 4 * tr + r;
      rvs[r] = rowB + lr < rows ? *(const uint4 *)(e.res + s_r[lr] + n) : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int lr = 4 * tr + r;
    if (rowB + lr >= rows) break;
    h2 v[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
      if (MB && nblk > 1) {
        v[p] = (h2){f2h(fb[MB ? r : 0][MB ? 2 * p : 0] + bias32[2 * p]),
                    f2h(fb[MB ? r : 0][MB ? 2 * p + 1 : 0] + bias32[2 * p + 1])};
      } else {
        v[p] = acc[r][p] + (h2){hfrom(bias16[2 * p]), hfrom(bias16[2 * p + 1])};
      }
      if (e.act == 1) v[p] = silu2_lut(v[p], s_t01, s_t2);
      else if (e.act == 2) v[p] = (h2){hmax(v[p].x, (h16)0.0f), hmax(v[p].y, (h16)0.0f)};
    }
    if (full) {
      if (e.res) {
        const uint4 rv = RES ? rvs[r] : *(const uint4 *)(e.res + s_r[lr] + n);
        v[0] = v[0] + __builtin_bit_cast(h2, rv.x);
        v[1] = v[1] + __builtin_bit_cast(h2, rv.y);
        v[2] = v[2] + __builtin_bit_cast(h2, rv.z);
        v[3] = v[3] + __builtin_bit_cast(h2, rv.w);
      }
      *(uint4 *)(e.out + s_o[lr] + n) =
          make_uint4(__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                     __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3]));
    } else {
#pragma unroll
      for (int c = 0; c < 8; c++) {
        if (n + c >= nend) break;
        h16 x = (c & 1) ? v[c >> 1].y : v[c >> 1].x;
        if (e.res) x = x + hfrom(e.res[s_r[lr] + n + c]);
        e.out[s_o[lr] + n + c] = hbits(x);
      }
    }
  }
}

// The split form's second kernel: per output the K blocks' fp16 results summed in fp32 in block order from +0 (the
// reference's flush_add), + the fp32 bias, one rounding to fp16, the activation, the residual, the (padded) store.
// A thread per row and 8 channels.
template <bool VEC>
__global__ __launch_bounds__(256) void k_gemm_f16c(const uint16_t *__restrict__ part, int nsplit, long long rows, int M,
                                                   double rM, const float *__restrict__ b32, int Np, Epi16Dev e) {
  __shared__ uint32_t s_t01[16];
  __shared__ uint16_t s_t2[16];
  if (threadIdx.x < 16) {
    s_t01[threadIdx.x] = (uint32_t)k_silu_c0[threadIdx.x] | ((uint32_t)k_silu_c1[threadIdx.x] << 16);
    s_t2[threadIdx.x] = k_silu_c2[threadIdx.x];
  }
  __syncthreads();
  const int np8 = Np / 8;
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * np8) return;
  const long long row = i / np8;
  const int n = (int)(i - row * np8) * 8;
  float fb[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int si = 0; si < nsplit; si++) {
    const uint4 q = *(const uint4 *)(part + ((long long)si * rows + row) * Np + n);
    const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const h2 hv = __builtin_bit_cast(h2, w4[j]);
      fb[2 * j] = fb[2 * j] + (float)hv.x;
      fb[2 * j + 1] = fb[2 * j + 1] + (float)hv.y;
    }
  }
  const int w = bnh_div(row, M, rM), m = (int)(row - (long long)w * M);
  long long orow = m;
  if (e.opad) {
    const int y = m / e.ow;
    orow = (long long)(y + e.opad) * (e.ow + 2 * e.opad) + (m - y * e.ow) + e.opad;
  }
  uint16_t *o = e.out + w * e.out_ws + orow * e.ldo + n;
  const uint16_t *rp = e.res ? e.res + w * e.res_ws + (long long)m * e.ldr + n : nullptr;
  h2 v[4];
#pragma unroll
  for (int p = 0; p < 4; p++) {
    v[p] = (h2){f2h(fb[2 * p] + b32[n + 2 * p]), f2h(fb[2 * p + 1] + b32[n + 2 * p + 1])};
    if (e.act == 1) v[p] = silu2_lut(v[p], s_t01, s_t2);
    else if (e.act == 2) v[p] = (h2){hmax(v[p].x, (h16)0.0f), hmax(v[p].y, (h16)0.0f)};
  }
  if (VEC) {
    if (rp) {
      const uint4 rv = *(const uint4 *)rp;
      v[0] = v[0] + __builtin_bit_cast(h2, rv.x);
      v[1] = v[1] + __builtin_bit_cast(h2, rv.y);
      v[2] = v[2] + __builtin_bit_cast(h2, rv.z);
      v[3] = v[3] + __builtin_bit_cast(h2, rv.w);
    }
    *(uint4 *)o = make_uint4(__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                             __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3]));
  } else {
#pragma unroll
    for (int c = 0; c < 8; c++) {
      h16 x = (c & 1) ? v[c >> 1].y : v[c >> 1].x;
      if (rp) x = x + hfrom(rp[c]);
      o[c] = hbits(x);
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
  uint16_t *hw = (uint16_t *)calloc((size_t)Nt * Kp, 2), *hwk = (uint16_t *)calloc((size_t)Nt * Kp, 2);
  uint16_t *hb16 = (uint16_t *)calloc(Nt, 2);
  float *hb = (float *)calloc(Nt, 4);
  bnh_h16w *W = (bnh_h16w *)calloc(1, sizeof *W);
  if (!hw || !hwk || !hb || !hb16 || !W) {
    free(hw); free(hwk); free(hb); free(hb16); free(W);
    bnh_fail("bnh_h16w_new: out of host memory");
    return nullptr;
  }
  for (int n = 0; n < Np; n++)  // hp_pack's layout (src/gemm_f16.c:18-40)
    for (int k = 0; k < Kp; k++) {
      const int nb = n / 16;
      const size_t idx = nb < n16 ? ((size_t)nb * Kp + k) * 16 + n % 16 : (size_t)n16 * Kp * 16 + (size_t)k * 8 + n % 16;
      hw[(size_t)n * Kp + k] = w[idx];
      hwk[(size_t)k * Nt + n] = w[idx];
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
  bool ok = (W->w = (uint16_t *)bnh_malloc((size_t)Nt * Kp * 2)) && (W->wk = (uint16_t *)bnh_malloc((size_t)Nt * Kp * 2)) &&
            (W->b = (float *)bnh_malloc(4 * (size_t)Nt)) && (W->b16 = (uint16_t *)bnh_malloc(2 * (size_t)Nt)) &&
            !bnh_memcpy_h2d(W->w, hw, (size_t)Nt * Kp * 2) && !bnh_memcpy_h2d(W->wk, hwk, (size_t)Nt * Kp * 2) &&
            !bnh_memcpy_h2d(W->b, hb, 4 * (size_t)Nt) && !bnh_memcpy_h2d(W->b16, hb16, 2 * (size_t)Nt);
  free(hw); free(hwk); free(hb); free(hb16);
  if (!ok) { bnh_h16w_free(W); return nullptr; }
  return W;
}

void bnh_h16w_free(bnh_h16w *W) {
  if (!W) return;
  if (W->w) (void)hipFree(W->w);
  if (W->wk) (void)hipFree(W->wk);
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

size_t bnh_gemm_f16_ws_bytes(int M, int B, const bnh_h16w *W) {
  if (!W || M <= 0 || B <= 0) return 0;
  const int nblk = (W->Kp + 127) / 128;
  return nblk > 1 ? (size_t)nblk * M * B * W->Np * 2 : 0;
}

static int gemm_f16e_run(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W,
                         const bnh_epi16 *e, const uint16_t *gh, long long gh_ws, void *ws, size_t ws_bytes,
                         void *stream) {
  if (gemm_f16_check(A, a_ws, lda, M, B, W, e)) return -1;
  BNH_REQ(!gh || (((uintptr_t)gh & 15) == 0 && (B == 1 || (gh_ws >= W->Kp && gh_ws % 8 == 0))));
  BNH_REQ(!ws || ((uintptr_t)ws & 15) == 0);
  const long long rows = (long long)M * B;
  Epi16Dev d = {e->act, e->out, e->out_ws, e->ldo, e->ow, e->opad, e->res, e->res_ws, e->ldr};
  const int nblk = (W->Kp + 127) / 128, bs = ((W->Kp + nblk - 1) / nblk + 7) & ~7;  // kblocks (src/gemm_f16.c:55-58)
  // channel tiles: as few as cover Np with at most 128 channels each, TC = Np / 8 spread over them (at least 4)
  const int np8 = W->Np / 8, ntile = (np8 + 15) / 16;
  int tc = (np8 + ntile - 1) / ntile;
  if (tc < 4) tc = 4;
  const bool vec = ((uintptr_t)e->out & 15) == 0 && e->ldo % 8 == 0 && (B == 1 || e->out_ws % 8 == 0) &&
                   (!e->res || (((uintptr_t)e->res & 15) == 0 && e->ldr % 8 == 0 && (B == 1 || e->res_ws % 8 == 0)));
  const int tr = 256 / tc < 64 ? 256 / tc : 64, bm = 4 * tr;
  const long long nb = bnh_ceil_div(rows, bm) * bnh_ceil_div(W->Np, 8 * tc);
  // fewer than two blocks per CU and several K blocks: one block per K block, then the combining kernel
  const bool split = nblk > 1 && nb < 512 && ws && ws_bytes >= bnh_gemm_f16_ws_bytes(M, B, W);
  const int nsplit = split ? nblk : 1;
  uint16_t *part = split ? (uint16_t *)ws : nullptr;
  BNH_REQ(nb * nsplit < (1LL << 31) && rows * np8 < (1LL << 40));
  const dim3 grid((unsigned)(nb * nsplit));
  hipStream_t st = bnh_stream(stream);
  const bool mb = nblk > 1 && !split;  // a block sums several K blocks
#define GEMM_F16E_(V_, R_, G_, M_)                                                                                     \
  hipLaunchKernelGGL((k_gemm_f16e<V_, R_, G_, M_>), grid, dim3(256), 0, st, A, a_ws, lda, M, 1.0 / M, rows, W->wk,     \
                     W->Nt, W->b, W->b16, W->Kp, W->Np, bs, tc, d, gh, gh_ws, part, nsplit)
#define GEMM_F16E(V_, R_, G_)                                                                                          \
  do {                                                                                                                 \
    if (mb) GEMM_F16E_(V_, R_, G_, true);                                                                              \
    else GEMM_F16E_(V_, R_, G_, false);                                                                                \
  } while (0)
  if (gh) {
    if (vec && e->res && !split) GEMM_F16E(true, true, true);
    else if (vec) GEMM_F16E(true, false, true);
    else GEMM_F16E(false, false, true);
  } else {
    if (vec && e->res && !split) GEMM_F16E(true, true, false);
    else if (vec) GEMM_F16E(true, false, false);
    else GEMM_F16E(false, false, false);
  }
#undef GEMM_F16E
#undef GEMM_F16E_
  BNH_HIP(hipGetLastError());
  if (split) {
    const dim3 g2((unsigned)bnh_ceil_div(rows * np8, 256));
    if (vec)
      hipLaunchKernelGGL((k_gemm_f16c<true>), g2, dim3(256), 0, st, part, nsplit, rows, M, 1.0 / M, W->b, W->Np, d);
    else
      hipLaunchKernelGGL((k_gemm_f16c<false>), g2, dim3(256), 0, st, part, nsplit, rows, M, 1.0 / M, W->b, W->Np, d);
    BNH_HIP(hipGetLastError());
  }
  return 0;
}

int bnh_gemm_f16_ws(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W, const bnh_epi16 *e,
                    void *ws, size_t ws_bytes, void *stream) {
  return gemm_f16e_run(A, a_ws, lda, M, B, W, e, nullptr, 0, ws, ws_bytes, stream);
}

int bnh_gemm_f16_gated_ws(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W,
                          const bnh_epi16 *e, const uint16_t *gh, long long gh_ws, void *ws, size_t ws_bytes,
                          void *stream) {
  BNH_REQ(gh);
  return gemm_f16e_run(A, a_ws, lda, M, B, W, e, gh, gh_ws, ws, ws_bytes, stream);
}

int bnh_gemm_f16_body(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W, const bnh_epi16 *e,
                      void *stream) {
  return bnh_gemm_f16_ws(A, a_ws, lda, M, B, W, e, nullptr, 0, stream);
}

int bnh_gemm_f16(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W, const bnh_epi16 *e,
                 void *stream) {
  if (gemm_f16_check(A, a_ws, lda, M, B, W, e) || zero_halo16(e, M, B, stream)) return -1;
  return bnh_gemm_f16_body(A, a_ws, lda, M, B, W, e, stream);
}

static int gemm_f16_mfma_run(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W,
                             const bnh_epi16 *e, const uint16_t *gh, long long gh_ws, bool zero, void *stream) {
  if (gemm_f16_check(A, a_ws, lda, M, B, W, e) || (zero && zero_halo16(e, M, B, stream))) return -1;
  BNH_REQ(!gh || (((uintptr_t)gh & 15) == 0 && (B == 1 || (gh_ws % 8 == 0 && gh_ws >= W->Kp))));
  BNH_REQ(lda % 8 == 0 && ((uintptr_t)A & 15) == 0 && (B == 1 || a_ws % 8 == 0));
  const long long rows = (long long)M * B;
  Epi16Dev d = {e->act, e->out, e->out_ws, e->ldo, e->ow, e->opad, e->res, e->res_ws, e->ldr};
  // 16-byte row chunks: 8-channel aligned rows in both the output and the residual
  const bool vec = ((uintptr_t)e->out & 15) == 0 && e->ldo % 8 == 0 && (B == 1 || e->out_ws % 8 == 0) &&
                   (!e->res || (((uintptr_t)e->res & 15) == 0 && e->ldr % 8 == 0 && (B == 1 || e->res_ws % 8 == 0))) &&
                   W->Np % 8 == 0;
  const long long nblocks = bnh_ceil_div(rows, 64) * bnh_ceil_div(W->Np, 128);
  BNH_REQ(nblocks < (1LL << 31));
  const dim3 grid((unsigned)nblocks);
  const double rM = 1.0 / M;
#define F16M_LAUNCH(G, V)                                                                                          \
  hipLaunchKernelGGL((k_gemm_f16<G, V>), grid, dim3(256), 0, bnh_stream(stream), A, a_ws, lda, M, rM, rows, W->w, \
                     W->b, W->Kp, W->Np, d, gh, gh_ws)
  if (gh) {
    if (vec) F16M_LAUNCH(true, true);
    else F16M_LAUNCH(true, false);
  } else {
    if (vec) F16M_LAUNCH(false, true);
    else F16M_LAUNCH(false, false);
  }
#undef F16M_LAUNCH
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_gemm_f16_mfma(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W, const bnh_epi16 *e,
                      void *stream) {
  return gemm_f16_mfma_run(A, a_ws, lda, M, B, W, e, nullptr, 0, true, stream);
}
// the op's form: the PW op zeroes the output halo itself, only when its buffer does not keep it
int bnh_gemm_f16_mfma_body(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W,
                           const bnh_epi16 *e, const uint16_t *gh, long long gh_ws, void *stream) {
  return gemm_f16_mfma_run(A, a_ws, lda, M, B, W, e, gh, gh_ws, false, stream);
}

int bnh_gemm_f16_mfma_gated(const uint16_t *A, long long a_ws, int lda, int M, int B, const bnh_h16w *W,
                            const bnh_epi16 *e, const uint16_t *gh, long long gh_ws, void *stream) {
  BNH_REQ(gh);
  return gemm_f16_mfma_run(A, a_ws, lda, M, B, W, e, gh, gh_ws, true, stream);
}

}  // extern "C"
