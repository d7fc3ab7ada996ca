// The int8 prototype head of libbnneon (PROTO_S8: src/proto_s8n.c, src/rt_ops_s8n.c:212-253, src/pc_kern_f32.c:364-374)
// on gfx950: per-cell symmetric int8 quantization of the L2-normalised cells, the cells x prototypes int8 MFMA GEMM
// whose epilogue keeps only the column maxima over each window's cells, and the class logits. Bit-identical to the
// reference (exact int32 sums; the max is exact and order-free; every float op as the reference rounds it).
//
// Prototypes are repacked at load from [Np/4][Kp/16][4][16] into K-blocks of 16 prototypes x 64 channels (1 KB each,
// prototype-group-major), zero past Np (rounded up to 256) and Kp (rounded up to 64). Two column-max kernels: k_proto_gemm64, the batched GEMM over every window's cells at once (64 cells
// per window), and k_proto_colmax, one window per block, for other cell counts.
#include <stdlib.h>
#include <string.h>

#include "bnh_internal.h"
#include "bnh_lds_dma.h"
#include "bnh_num.h"

typedef int v4i __attribute__((ext_vector_type(4)));

struct bnh_s8p {
  int Np, Kp, Npt, Kt;  // Npt = Np rounded up to 256, Kt = Kp rounded up to 64
  int8_t *w;            // K-blocked: prototype n, byte k at ((n / 16) (Kt / 64) + k / 64) 1024 + (n % 16) 64 + k % 64,
                        // zero past Np and Kp
  float *sw;            // [Npt]
};
// byte offset of prototype n, channel k in the K-blocked rows
static inline size_t s8p_at(int n, int k, int Kt) {
  return ((size_t)(n >> 4) * (Kt >> 6) + (k >> 6)) * 1024 + (n & 15) * 64 + (k & 63);
}

// ------------------------------------------------------------------ cell quantization (pc_quant_cells_f32)
// One wave per cell. The reference's sum of squares is 8 fused chains (channel c feeds chain c % 8, in order of c):
// lanes 0..7 run them over a 512-float LDS chunk the whole wave stages, then combine as ((t0 + t1) + (t2 + t3)),
// t_j = chain_j + chain_{j+4}. max |x| (FMAX, NaN-propagating) is order-free: all lanes, then a wave reduction.
#define QC_CHUNK 512
// F16: the cells are fp16 (pc_quant_cells_f16, src/pc_proto_s8.c:14-45: the same sums of the widened values, and
// codes narrowed with saturation to [-128, 127] without the floor at -127)
template <bool F16>
__global__ __launch_bounds__(256) void k_quant_cells(const void *__restrict__ xv, long long x_ws, int P, int C, int ld,
                                                     float eps, int8_t *__restrict__ qa, long long qa_ws, int Kp,
                                                     float *__restrict__ sx, long long sx_ws, long long cells) {
  __shared__ float stage[4][QC_CHUNK];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const long long cell = (long long)blockIdx.x * 4 + wv;
  const bool live = cell < cells;
  const int w = live ? (int)(cell / P) : 0, p = live ? (int)(cell % P) : 0;
  const float *r = F16 ? nullptr : (const float *)xv + w * x_ws + (long long)p * ld;
  const _Float16 *rh = F16 ? (const _Float16 *)xv + w * x_ws + (long long)p * ld : nullptr;
  float chain = 0.f, mx = 0.f;
  for (int c0 = 0; c0 < C; c0 += QC_CHUNK) {
    const int n = C - c0 < QC_CHUNK ? C - c0 : QC_CHUNK;
    if (live)
      for (int i = lane; i < n; i += 64) {
        const float v = F16 ? (float)rh[c0 + i] : r[c0 + i];
        stage[wv][i] = v;
        mx = bnh_fmax(mx, __builtin_fabsf(v));
      }
    __syncthreads();
    if (live && lane < 8)
      for (int i = lane; i < n; i += 8) chain = __builtin_fmaf(stage[wv][i], stage[wv][i], chain);
    __syncthreads();
  }
  if (!live) return;
  for (int off = 32; off; off >>= 1) mx = bnh_fmax(mx, __shfl_xor(mx, off));
  // lanes 0..3 hold chains j (channels 8i + j), lanes 4..7 chains j + 4: t_j = s0_j + s1_j
  const float s1 = __shfl(chain, (lane & 3) + 4);
  const float t = chain + s1;  // valid in lanes 0..3
  const float t0 = __shfl(t, 0), t1 = __shfl(t, 1), t2 = __shfl(t, 2), t3 = __shfl(t, 3);
  const float den = __builtin_sqrtf((t0 + t1) + (t2 + t3)) + eps;
  if (!(mx > 0)) mx = 1e-30f;
  if (lane == 0) sx[w * sx_ws + p] = mx / (127.f * den);
  const float inv = 127.f / mx;
  int8_t *q = qa + w * qa_ws + (long long)p * Kp;
  for (int c = lane * 4; c < Kp; c += 256) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int32_t b = 0;
      if (c + j < C) {
        int32_t v = bnh_cvta_s32((F16 ? (float)rh[c + j] : r[c + j]) * inv);
        v = v < -32768 ? -32768 : v > 32767 ? 32767 : v;
        v = v < -128 ? -128 : v > 127 ? 127 : v;
        b = F16 || v >= -127 ? v : -127;
      }
      word |= ((uint32_t)b & 0xffu) << (8 * j);
    }
    *(uint32_t *)(q + c) = word;
  }
}

// ------------------------------------------------------------------ column maxima (pc_proto_colmax_s8n)
BNH_DEV float wave16_max_cols(float v) {  // max over lane groups l>>4 (lanes l, l^16, l^32, l^48)
  v = bnh_fmax(v, __shfl_xor(v, 16));
  v = bnh_fmax(v, __shfl_xor(v, 32));
  return v;
}

__global__ __launch_bounds__(256) void k_proto_colmax(const int8_t *__restrict__ qa, long long qa_ws, int Kp,
                                                      const float *__restrict__ sx, long long sx_ws, int P,
                                                      const int8_t *__restrict__ wt, const float *__restrict__ sw,
                                                      int Np, float *__restrict__ colmax, long long cm_ws) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int win = blockIdx.x;
  const int n0 = blockIdx.y * 256 + wv * 64;
  const int kc = (lane >> 4) * 16;
  const int8_t *aw = qa + win * qa_ws;
  const float *sxw = sx + win * sx_ws;
  const long long kblk = (long long)((Kp + 63) >> 6) * 1024;  // one 16-prototype group of the K-blocked rows
  const int8_t *bp = wt + (long long)(n0 >> 4) * kblk + (lane & 15) * 64 + kc;  // + j kblk + k / 64 1024
  float run[4] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  const int kmain = Kp & ~63;
  for (int r0 = 0; r0 < P; r0 += 64) {
    const int8_t *ap[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      int row = r0 + 16 * t + (lane & 15);
      if (row >= P) row = P - 1;  // valid memory; excluded from the max below
      ap[t] = aw + (long long)row * Kp + kc;
    }
    v4i acc[4][4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[t][j] = (v4i){0, 0, 0, 0};
    for (int k = 0; k < kmain; k += 64) {
      v4i a[4], b[4];
#pragma unroll
      for (int t = 0; t < 4; t++) a[t] = *(const v4i *)(ap[t] + k);
#pragma unroll
      for (int j = 0; j < 4; j++) b[j] = *(const v4i *)(bp + j * kblk + (k >> 6) * 1024);
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[t][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[j], acc[t][j], 0, 0, 0);
    }
    if (kmain < Kp) {
      const bool in = kmain + kc < Kp;
      v4i a[4], b[4];
#pragma unroll
      for (int t = 0; t < 4; t++) a[t] = in ? *(const v4i *)(ap[t] + kmain) : (v4i){0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < 4; j++) b[j] = in ? *(const v4i *)(bp + j * kblk + (kmain >> 6) * 1024) : (v4i){0, 0, 0, 0};
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[t][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[j], acc[t][j], 0, 0, 0);
    }
    // acc[t][j][r]: cell r0 + 16t + 4(lane>>4) + r, prototype n0 + 16j + (lane&15)
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = r0 + 16 * t + 4 * (lane >> 4) + r;
        if (row >= P) continue;
        const float s = sxw[row];
#pragma unroll
        for (int j = 0; j < 4; j++) run[j] = bnh_fmax(run[j], (float)acc[t][j][r] * s);
      }
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const float m = wave16_max_cols(run[j]);
    const int n = n0 + 16 * j + (lane & 15);
    if (lane < 16 && n < Np) colmax[win * cm_ws + n] = m * sw[n];
  }
}

// ------------------------------------------------------------------ column maxima as one batched GEMM
// The cells of all windows (64 per window: rows win * 64 + p of the product) times all prototypes, K = Kp, in tiles
// of 256 cells (4 windows) x 256 prototypes. Persistent blocks, one per CU; 4 waves of 128 cells (2 windows) x 128
// prototypes = 8 x 8 i8 MFMA tiles each (256 accumulators in AGPRs). The K slices (64 bytes of k) of every tile a
// block owns form one 4-stage LDS ring (32 KB a stage) fed by direct global -> LDS loads issued three slices ahead,
// so a tile's epilogue runs while the next tile's first slices load. In LDS both operands are [row][64 bytes] with
// XOR-swizzled 16-byte chunks (chunk c of row r at r * 64 + 16 (c ^ ((r >> 1) & 3))): a DMA instruction's 64 lanes
// fill 16 whole rows, and the 16 rows one ds_read_b128 phase serves land on distinct banks. The prototypes are stored
// K-blocked (see bnh_s8p), so each of their DMA instructions reads 1 KB of contiguous memory.
//
// Tile order: the tile grid (cell tiles x prototype tiles) is cut into 8 regions, one per XCD (blocks b, b + 8, ...
// run on XCD b % 8), 8 x 1 when there are at least 8 cell tiles (each XCD's cells stay in its L2 while it streams every
// prototype once), fewer cell parts and more prototype parts for small batches. Within a region the tiles go
// prototype-major, and the blocks of an XCD run through the same K slices at about the same time, so a slice one
// block fetches is an L2 hit for the others.
//
// Epilogue (pc_proto_colmax_s8n, src/proto_s8n.c:139-164): per window and prototype, the maximum over the window's 64
// cells of (float)acc * sx (one rounding each; the maximum is exact and order-free), times sw. The maximum is the
// IEEE 754-2019 maximum (v_maximum3_f32, two elements per instruction): like the reference's FMAX it returns NaN when
// either operand is NaN and orders -0 below +0; only the payload of a NaN may differ (such a window fails either way).
// The tile's 256 cell scales and 256 prototype scales reach LDS by DMA with the tile's first K slice
// (double-buffered by tile parity).
#define PG_TM 256
#define PG_TN 256
#define PG_BK 64
#define PG_AB (PG_TM * PG_BK)
#define PG_STAGE (PG_AB + PG_TN * PG_BK)
#define PG_NST 4
#define PG_SCL (PG_NST * PG_STAGE)  // 2 x (256 sx + 256 sw) floats after the ring
typedef __attribute__((address_space(3))) v4i lds_v4i;
typedef __attribute__((address_space(3))) float lds_f32;

BNH_DEV float pg_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }
// the maximum of lanes l, l ^ 16, l ^ 32 and l ^ 48 (gfx950 row swaps: no LDS traffic)
BNH_DEV float pg_max16(float m) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  m = pg_max(__uint_as_float(r[0]), __uint_as_float(r[1]));  // rows (0, 1) and (2, 3)
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  return pg_max(__uint_as_float(q[0]), __uint_as_float(q[1]));  // halves (0, 1)
}
// an accumulator element read out of its AGPR where the epilogue uses it: without this the compiler copies all 256
// accumulators into VGPRs when the K loop ends and spills the block's other values to scratch
BNH_DEV int32_t pg_acc(int32_t x) {
  int32_t v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(x));
  return v;
}

// tile i of this block in its region: cell tile m_t, prototype tile n_t
struct PgRegion {
  int lid, nlb, m_lo, mx, n_lo;
  __device__ void tile(int i, int &m_t, int &n_t) const {
    const int u = lid + i * nlb;
    m_t = m_lo + u % mx;
    n_t = n_lo + u / mx;
  }
};

__global__ __launch_bounds__(256, 1) void k_proto_gemm64(const int8_t *__restrict__ qa, long long qa_ws,
                                                        const float *__restrict__ sx, long long sx_ws, int B, int Kp,
                                                        const int8_t *__restrict__ wt, const float *__restrict__ sw,
                                                        int Np, int n_mt, int n_nt, float *__restrict__ colmax,
                                                        long long cm_ws) {
  __shared__ __attribute__((aligned(1024))) int8_t lds_raw[PG_SCL + 2 * 2048];
  lds_i8 *lds = (lds_i8 *)lds_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  // this block's region of the tile grid and its tiles in it
  const int xcd = (int)(blockIdx.x & 7);
  PgRegion R;
  R.lid = (int)(blockIdx.x >> 3);
  R.nlb = (int)(gridDim.x >> 3);
  const int gm = n_mt >= 8 ? 8 : n_mt >= 4 ? 4 : n_mt >= 2 ? 2 : 1, gn = 8 / gm;
  const int rm = xcd / gn, rn = xcd % gn;
  R.m_lo = rm * n_mt / gm;
  R.mx = (rm + 1) * n_mt / gm - R.m_lo;
  R.n_lo = rn * n_nt / gn;
  const int nx = (rn + 1) * n_nt / gn - R.n_lo;
  const int xtiles = R.mx * nx;
  const int mytiles = xtiles > R.lid ? (xtiles - 1 - R.lid) / R.nlb + 1 : 0;
  const int steps = Kp / PG_BK;
  // DMA lane roles: an instruction fills 16 rows of 64 bytes, lane -> row lane / 4, its 16-byte slot lane % 4
  // holding k chunk (lane % 4) ^ ((lane / 8) % 4). Per K slice a wave issues 4 cell instructions (rows 64 wave ..
  // 64 wave + 63 of the tile: window m_t 4 + wave) and 4 prototype instructions (rows 64 wave .. 64 wave + 63).
  const int dchunk = 16 * ((lane & 3) ^ ((lane >> 3) & 3));
  const uint32_t loff_a = (uint32_t)((lane >> 2) * Kp + dchunk);  // cell rows: Kp apart
  const uint32_t loff_b = (uint32_t)((lane >> 2) * PG_BK + dchunk);  // a K-blocked 16-row group: 64 bytes apart
  const long long a16 = 16LL * Kp, b16 = (long long)(Kp / PG_BK) * 1024;  // the next 16 rows of each operand
  // Issue state, advanced incrementally (the scalar unit is shared by the CU's waves): the next (tile, K step) to
  // issue, the stage it fills, and the tile's operand bases.
  int iss_i = 0, iss_k = 0, iss_st = 0;
  const int8_t *a_tile = qa, *b_tile = wt;
  auto issue = [&]() {
    if (iss_k == 0) {  // a new tile: its operand bases and scales
      int m_t, n_t;
      R.tile(iss_i, m_t, n_t);
      int win = m_t * 4 + wave;
      if (win > B - 1) win = B - 1;  // cells past the last window: valid memory, results dropped
      a_tile = qa + (long long)win * qa_ws;
      b_tile = wt + (long long)(n_t * 16 + 4 * wave) * b16;
      if (wave < 2) {  // the tile's scales: wave 0 the cell scales, wave 1 the prototype scales
        lds_i8 *sc = lds + PG_SCL + (iss_i & 1) * 2048 + wave * 1024;
        if (wave == 0) {
          const int last = B - 1 - m_t * 4;  // windows past the last one read the last window's scales (unused)
          const int wl = (lane >> 4) < last ? (lane >> 4) : last;
          rq_dma16s(sx + (long long)m_t * 4 * sx_ws, (uint32_t)(wl * sx_ws * 4 + 16 * (lane & 15)), sc);
        } else {
          rq_dma16s(sw + n_t * PG_TN, (uint32_t)(16 * lane), sc);
        }
      }
    }
    lds_i8 *st = lds + iss_st * PG_STAGE;
    const int8_t *ab = a_tile + iss_k * PG_BK, *bb = b_tile + iss_k * 1024;
#pragma unroll
    for (int h = 0; h < 4; h++) rq_dma16s(ab + h * a16, loff_a, st + (4 * wave + h) * 1024);
#pragma unroll
    for (int h = 0; h < 4; h++) rq_dma16s(bb + h * b16, loff_b, st + PG_AB + (4 * wave + h) * 1024);
    if (++iss_st == PG_NST) iss_st = 0;
    if (++iss_k == steps) { iss_k = 0; iss_i++; }
  };
  // fragment reads: row r of a stage's operand at r * 64 + 16 (chunk ^ ((r >> 1) & 3)); for the rows 16 t + (lane & 15)
  // of a wave's tile the swizzle depends on the lane only, so tile t is an immediate offset t * 1024
  const int g = lane >> 4, j16 = lane & 15;
  const int foff = j16 * PG_BK + 16 * (g ^ ((j16 >> 1) & 3));
  const int fa_off = wm * 128 * PG_BK + foff, fb_off = PG_AB + wn * 128 * PG_BK + foff;
  const int total = mytiles * steps;
  for (int gs = 0; gs < PG_NST - 1 && gs < total; gs++) issue();
  int gs = 0, cst = 0;  // the global step being computed and its stage
  for (int ci = 0; ci < mytiles; ci++) {
    v4i acc[8][8];
#pragma unroll
    for (int t = 0; t < 8; t++)
#pragma unroll
      for (int jj = 0; jj < 8; jj++) acc[t][jj] = (v4i){0, 0, 0, 0};
    for (int ck = 0; ck < steps; ck++, gs++) {
      // this wave's loads of step gs have landed once at most those of the two later steps (8 a step) are
      // outstanding; the scale loads and the epilogue's stores only make the wait longer
      if (gs + 2 < total) RQ_WAIT_VM(16);
      else if (gs + 1 < total) RQ_WAIT_VM(8);
      else RQ_WAIT_VM(0);
      RQ_BARRIER();  // every wave's loads of step gs have landed; the stage of step gs - 1 is no longer read
      if (gs + PG_NST - 1 < total) issue();
      const lds_i8 *st = lds + cst * PG_STAGE;
      if (++cst == PG_NST) cst = 0;
      const lds_i8 *pa = st + fa_off, *pb = st + fb_off;
      v4i a[8], b[8];
#pragma unroll
      for (int t = 0; t < 8; t++) a[t] = *(const lds_v4i *)(pa + t * 1024);
#pragma unroll
      for (int jj = 0; jj < 8; jj++) b[jj] = *(const lds_v4i *)(pb + jj * 1024);
#pragma unroll
      for (int jj = 0; jj < 8; jj++)
#pragma unroll
        for (int t = 0; t < 8; t++) acc[t][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[jj], acc[t][jj], 0, 0, 0);
    }
    // ---- epilogue: acc[t][jj][r] is cell row 16 (t % 4) + 4 g + r of window m_t 4 + 2 wm + t / 4, prototype
    // wn 128 + 16 jj + j16 of the tile
    int m_t, n_t;
    R.tile(ci, m_t, n_t);
    const lds_f32 *sxs = (const lds_f32 *)(lds + PG_SCL + (ci & 1) * 2048);
    const lds_f32 *sws = sxs + 256;
#pragma unroll
    for (int wl = 0; wl < 2; wl++) {
      float srow[4][4];
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) srow[t][r] = sxs[wm * 128 + 64 * wl + 16 * t + 4 * g + r];
      const int win = m_t * 4 + wm * 2 + wl;
#pragma unroll
      for (int jj = 0; jj < 8; jj++) {
        float m = -__builtin_inff();
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
          for (int r = 0; r < 4; r++) m = pg_max(m, (float)pg_acc(acc[4 * wl + t][jj][r]) * srow[t][r]);
        m = pg_max(m, __shfl_xor(m, 16));
        m = pg_max(m, __shfl_xor(m, 32));
        const int nl = wn * 128 + 16 * jj + j16, n = n_t * PG_TN + nl;
        if (lane < 16 && win < B && n < Np) colmax[win * cm_ws + n] = m * sws[nl];
      }
    }
  }
}

// The same GEMM with 8 waves in two ping-pong groups. Waves 0-3 (group 0) and 4-7 (group 1) put one wave of each
// group on every SIMD; the wave of group g owns cells 128 g .. 128 g + 127 (2 windows) x prototypes 64 (wave % 4) ..
// + 63 of the tile (8 x 4 MFMA tiles, 128 accumulators). Every K slice is a memory phase (issue the DMA three slices
// ahead, read the slice's 12 fragments into registers) then a compute phase (32 MFMAs, and the epilogue after a tile's
// last slice), with a block barrier after each phase. Group 1 starts one barrier late, so between any two barriers one
// group reads LDS while the other runs MFMAs: the matrix cores of a SIMD are fed by one wave while the other waits
// on its fragment reads.
//   Slice s is read by group 0 in interval 2s and by group 1 in interval 2s + 1 (interval i lies between barrier i and
// barrier i + 1). Every wave waits for its own DMA of slice s + 1 (vmcnt) before the barrier that opens interval
// 2s + 2, and for its fragment reads (lgkmcnt) before the barrier that ends its memory phase; the DMA of slice s + 3
// issued in interval 2s (group 0) or 2s + 1 (group 1) refills the stage of slice s - 1, whose last reads were in
// interval 2s - 1. The tile's scales use the same double buffer as the 4-wave kernel (K slices >= 4).
BNH_DEV void pp_sync() {
  __builtin_amdgcn_sched_barrier(0);  // no instruction moves across a phase boundary
  RQ_BARRIER();
  __builtin_amdgcn_sched_barrier(0);
}
// this wave's DMA of slice s + 1 has landed: at most the loads of the (up to two) slices issued after it are pending
BNH_DEV void pp_wait_next(int total, int s) {
  const int later = total - 2 - s;
  if (later >= 2) RQ_WAIT_VM(8);
  else if (later == 1) RQ_WAIT_VM(4);
  else RQ_WAIT_VM(0);
}

__global__ __launch_bounds__(512, 1) void k_proto_gemm_pp(const int8_t *__restrict__ qa, long long qa_ws,
                                                         const float *__restrict__ sx, long long sx_ws, int B, int Kp,
                                                         const int8_t *__restrict__ wt, const float *__restrict__ sw,
                                                         int Np, int n_mt, int n_nt, float *__restrict__ colmax,
                                                         long long cm_ws) {
  __shared__ __attribute__((aligned(1024))) int8_t lds_raw[PG_SCL + 2 * 2048];
  lds_i8 *lds = (lds_i8 *)lds_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2, wn = wave & 3;
  const int xcd = (int)(blockIdx.x & 7);
  PgRegion R;
  R.lid = (int)(blockIdx.x >> 3);
  R.nlb = (int)(gridDim.x >> 3);
  const int gm = n_mt >= 8 ? 8 : n_mt >= 4 ? 4 : n_mt >= 2 ? 2 : 1, gn = 8 / gm;
  const int rm = xcd / gn, rn = xcd % gn;
  R.m_lo = rm * n_mt / gm;
  R.mx = (rm + 1) * n_mt / gm - R.m_lo;
  R.n_lo = rn * n_nt / gn;
  const int nx = (rn + 1) * n_nt / gn - R.n_lo;
  const int xtiles = R.mx * nx;
  const int mytiles = xtiles > R.lid ? (xtiles - 1 - R.lid) / R.nlb + 1 : 0;
  const int steps = Kp / PG_BK;
  // DMA roles: per K slice a wave issues 2 cell instructions (rows 32 wave .. 32 wave + 31 of the tile: cells
  // 32 (wave % 2) .. of window m_t 4 + wave / 2) and 2 prototype instructions (rows 32 wave .. 32 wave + 31)
  const int dchunk = 16 * ((lane & 3) ^ ((lane >> 3) & 3));
  const uint32_t loff_a = (uint32_t)((lane >> 2) * Kp + dchunk);
  const uint32_t loff_b = (uint32_t)((lane >> 2) * PG_BK + dchunk);
  const long long a16 = 16LL * Kp, b16 = (long long)(Kp / PG_BK) * 1024;
  int iss_i = 0, iss_k = 0, iss_st = 0;
  const int8_t *a_tile = qa, *b_tile = wt;
  auto issue = [&]() {
    if (iss_k == 0) {
      int m_t, n_t;
      R.tile(iss_i, m_t, n_t);
      int win = m_t * 4 + (wave >> 1);
      if (win > B - 1) win = B - 1;
      a_tile = qa + (long long)win * qa_ws + (long long)(wave & 1) * 32 * Kp;
      b_tile = wt + (long long)(n_t * 16 + 2 * wave) * b16;
      if (wave < 2) {
        lds_i8 *sc = lds + PG_SCL + (iss_i & 1) * 2048 + wave * 1024;
        if (wave == 0) {
          const int last = B - 1 - m_t * 4;
          const int wl = (lane >> 4) < last ? (lane >> 4) : last;
          rq_dma16s(sx + (long long)m_t * 4 * sx_ws, (uint32_t)(wl * sx_ws * 4 + 16 * (lane & 15)), sc);
        } else {
          rq_dma16s(sw + n_t * PG_TN, (uint32_t)(16 * lane), sc);
        }
      }
    }
    lds_i8 *st = lds + iss_st * PG_STAGE;
    const int8_t *ab = a_tile + iss_k * PG_BK, *bb = b_tile + iss_k * 1024;
#pragma unroll
    for (int h = 0; h < 2; h++) rq_dma16s(ab + h * a16, loff_a, st + (2 * wave + h) * 1024);
#pragma unroll
    for (int h = 0; h < 2; h++) rq_dma16s(bb + h * b16, loff_b, st + PG_AB + (2 * wave + h) * 1024);
    if (++iss_st == PG_NST) iss_st = 0;
    if (++iss_k == steps) { iss_k = 0; iss_i++; }
  };
  const int g = lane >> 4, j16 = lane & 15;
  const int foff = j16 * PG_BK + 16 * (g ^ ((j16 >> 1) & 3));
  const int fa_off = grp * 128 * PG_BK + foff, fb_off = PG_AB + wn * 64 * PG_BK + foff;
  const int total = mytiles * steps;
  for (int s = 0; s < PG_NST - 1 && s < total; s++) issue();
  if (total > 2) RQ_WAIT_VM(8);  // slice 0 has landed
  else if (total == 2) RQ_WAIT_VM(4);
  else RQ_WAIT_VM(0);
  pp_sync();
  if (grp) pp_sync();  // group 1 runs one phase behind group 0
  v4i acc[8][4];
  // the column maxima of tile i: acc[t][jj][r] is cell row 16 (t % 4) + 4 g + r of window m_t 4 + 2 grp + t / 4,
  // prototype wn 64 + 16 jj + j16 of the tile
  auto epilogue = [&](int i) {
    int m_t, n_t;
    R.tile(i, m_t, n_t);
    const lds_f32 *sxs = (const lds_f32 *)(lds + PG_SCL + (i & 1) * 2048);
    const lds_f32 *sws = sxs + 256;
#pragma unroll
    for (int wl = 0; wl < 2; wl++) {
      float srow[4][4];
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) srow[t][r] = sxs[grp * 128 + 64 * wl + 16 * t + 4 * g + r];
      const int win = m_t * 4 + grp * 2 + wl;
#pragma unroll
      for (int jj = 0; jj < 4; jj++) {
        float m = -__builtin_inff();
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
          for (int r = 0; r < 4; r++) m = pg_max(m, (float)acc[4 * wl + t][jj][r] * srow[t][r]);
        m = pg_max16(m);
        const int nl = wn * 64 + 16 * jj + j16, n = n_t * PG_TN + nl;
        if (lane < 16 && win < B && n < Np) colmax[win * cm_ws + n] = m * sws[nl];
      }
    }
  };
  int cst = 0, ci = 0, ck = 0;
  int done = -1;  // a tile whose sums are complete and whose epilogue has not run
  for (int s = 0; s < total; s++) {
    asm volatile("" : "+s"(done));  // opaque to the optimiser: no peeled first iteration (it would spill)
    // ---- memory phase of slice s: its DMA three slices ahead, its fragments, and (on a tile's first slice) the
    // previous tile's epilogue, whose VALU work runs beside the other group's MFMAs
    if (s + PG_NST - 1 < total) issue();
    if (done >= 0) {
      epilogue(done);
      done = -1;
    }
    const lds_i8 *st = lds + cst * PG_STAGE;
    if (++cst == PG_NST) cst = 0;
    const lds_i8 *pa = st + fa_off, *pb = st + fb_off;
    v4i a[8], b[4];
#pragma unroll
    for (int t = 0; t < 8; t++) a[t] = *(const lds_v4i *)(pa + t * 1024);
#pragma unroll
    for (int jj = 0; jj < 4; jj++) b[jj] = *(const lds_v4i *)(pb + jj * 1024);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (grp) pp_wait_next(total, s);
    pp_sync();
    // ---- compute phase of slice s
    if (ck == 0) {  // a tile's first slice starts its sums from zero
#pragma unroll
      for (int jj = 0; jj < 4; jj++)
#pragma unroll
        for (int t = 0; t < 8; t++)
          acc[t][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[jj], (v4i){0, 0, 0, 0}, 0, 0, 0);
    } else {
#pragma unroll
      for (int jj = 0; jj < 4; jj++)
#pragma unroll
        for (int t = 0; t < 8; t++)
          acc[t][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[jj], acc[t][jj], 0, 0, 0);
    }
    if (++ck == steps) {
      done = ci;
      ck = 0;
      ci++;
    }
    if (!grp) pp_wait_next(total, s);
    pp_sync();
  }
  if (done >= 0) epilogue(done);
  if (!grp) pp_sync();  // every wave passes the same number of barriers
}

// ------------------------------------------------------------------ class logits (pc_proto_logits)
__global__ void k_proto_logits(const float *__restrict__ colmax, long long cm_ws, const float *__restrict__ w,
                               const float *__restrict__ b, int nc, int ppc, float *__restrict__ logits, long long lg_ws,
                               int B, int *__restrict__ win_fail, int fail_code) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)nc * B) return;
  const int win = (int)(i / nc), c = (int)(i % nc);
  const float *cm = colmax + win * cm_ws + (long long)c * ppc;
  const float *wr = w + (long long)c * ppc;
  float s = 0.f;
  for (int q = 0; q < ppc; q++) {
    const float t = cm[q] * wr[q];
    s = s + t;
  }
  const float v = s + b[c];
  logits[win * lg_ws + c] = v;
  if (!(__builtin_fabsf(v) <= 3.0e38f) && win_fail) atomicCAS(win_fail + win, 0, fail_code);
}

// ================================================================== host side
extern "C" {

bnh_s8p *bnh_s8p_new(int Np, int Kp, const int8_t *qw, const float *sw) {
  if (Np <= 0 || Np % 4 || Kp <= 0 || Kp % 16 || !qw || !sw) {
    bnh_fail("bnh_s8p_new: Np %d Kp %d: expected Np a multiple of 4, Kp a multiple of 16, both tensors", Np, Kp);
    return nullptr;
  }
  const int Npt = (int)bnh_round_up(Np, 256), Kt = (int)bnh_round_up(Kp, 64);
  int8_t *hw = (int8_t *)calloc((size_t)Npt * Kt, 1);
  float *hs = (float *)calloc(Npt, 4);
  bnh_s8p *W = (bnh_s8p *)calloc(1, sizeof *W);
  if (!hw || !hs || !W) {
    free(hw); free(hs); free(W);
    bnh_fail("bnh_s8p_new: out of host memory");
    return nullptr;
  }
  const int kb = Kp / 16;
  for (int n = 0; n < Np; n++)
    for (int k = 0; k < Kp; k++) hw[s8p_at(n, k, Kt)] = qw[((size_t)(n / 4) * kb + k / 16) * 64 + (n % 4) * 16 + k % 16];
  memcpy(hs, sw, sizeof(float) * Np);
  W->Np = Np; W->Kp = Kp; W->Npt = Npt; W->Kt = Kt;
  bool ok = (W->w = (int8_t *)bnh_malloc((size_t)Npt * Kt)) && (W->sw = (float *)bnh_malloc(4 * (size_t)Npt)) &&
            !bnh_memcpy_h2d(W->w, hw, (size_t)Npt * Kt) && !bnh_memcpy_h2d(W->sw, hs, 4 * (size_t)Npt);
  free(hw);
  free(hs);
  if (!ok) { bnh_s8p_free(W); return nullptr; }
  return W;
}

void bnh_s8p_free(bnh_s8p *W) {
  if (!W) return;
  if (W->w) (void)hipFree(W->w);
  if (W->sw) (void)hipFree(W->sw);
  free(W);
}

int bnh_quant_cells(const float *x, long long x_ws, int P, int C, int ld, float eps, int8_t *qa, long long qa_ws,
                    int Kp, float *sx, long long sx_ws, int B, void *stream) {
  BNH_REQ(x && qa && sx && P > 0 && C > 0 && B > 0);
  BNH_REQ(C % 8 == 0 && C <= Kp && Kp % 16 == 0 && ld >= C);
  BNH_REQ(((uintptr_t)qa & 3) == 0 && qa_ws % 4 == 0);
  BNH_REQ(B == 1 || (qa_ws >= (long long)P * Kp && sx_ws >= P && x_ws >= (long long)(P - 1) * ld + C));
  const long long cells = (long long)P * B;
  hipLaunchKernelGGL(k_quant_cells<false>, dim3((unsigned)bnh_ceil_div(cells, 4)), dim3(256), 0, bnh_stream(stream), x,
                     x_ws, P, C, ld, eps, qa, qa_ws, Kp, sx, sx_ws, cells);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_quant_cells_f16(const uint16_t *x, long long x_ws, int P, int C, int ld, float eps, int8_t *qa,
                        long long qa_ws, int Kp, float *sx, long long sx_ws, int B, void *stream) {
  BNH_REQ(x && qa && sx && P > 0 && C > 0 && B > 0);
  BNH_REQ(C % 8 == 0 && C <= Kp && Kp % 16 == 0 && ld >= C);
  BNH_REQ(((uintptr_t)qa & 3) == 0 && qa_ws % 4 == 0);
  BNH_REQ(B == 1 || (qa_ws >= (long long)P * Kp && sx_ws >= P && x_ws >= (long long)(P - 1) * ld + C));
  const long long cells = (long long)P * B;
  hipLaunchKernelGGL(k_quant_cells<true>, dim3((unsigned)bnh_ceil_div(cells, 4)), dim3(256), 0, bnh_stream(stream), x,
                     x_ws, P, C, ld, eps, qa, qa_ws, Kp, sx, sx_ws, cells);
  BNH_HIP(hipGetLastError());
  return 0;
}

// the dotprod head's prototype panels [Np/12][K/4][12][4] (src/pc_proto_s8.c:4-6) into this library's layout
bnh_s8p *bnh_s8p_new_c12(int Np, int K, const int8_t *qw, const float *sw) {
  if (!qw || !sw || Np <= 0 || Np % 12 || K <= 0 || K % 4) {
    bnh_fail("bnh_s8p_new_c12: Np %d K %d: expected Np %% 12 == 0, K %% 4 == 0 and both tensors", Np, K);
    return nullptr;
  }
  const int Kp = (K + 15) & ~15, kb = Kp / 16;
  int8_t *q4 = (int8_t *)calloc((size_t)Np * Kp, 1);
  if (!q4) {
    bnh_fail("bnh_s8p_new_c12: out of host memory");
    return nullptr;
  }
  for (int n = 0; n < Np; n++)
    for (int k = 0; k < K; k++)
      q4[((size_t)(n / 4) * kb + k / 16) * 64 + (n % 4) * 16 + k % 16] =
          qw[((size_t)(n / 12) * (K / 4) + k / 4) * 48 + (n % 12) * 4 + k % 4];
  bnh_s8p *W = bnh_s8p_new(Np, Kp, q4, sw);
  free(q4);
  return W;
}

int bnh_proto_colmax(const int8_t *qa, long long qa_ws, const float *sx, long long sx_ws, int P, const bnh_s8p *W,
                     float *colmax, long long cm_ws, int B, void *stream) {
  BNH_REQ(qa && sx && W && colmax && P > 0 && B > 0);
  BNH_REQ(((uintptr_t)qa & 15) == 0 && qa_ws % 16 == 0);
  BNH_REQ(B == 1 || (qa_ws >= (long long)P * W->Kp && cm_ws >= W->Np && sx_ws >= P));
  // the batched GEMM: 64 cells per window, K in 64-byte slices (at least 4: the scale buffers are reused two tiles
  // later), 16-byte aligned cell scales
  const bool batched = P == 64 && W->Kp % PG_BK == 0 && W->Kp >= 4 * PG_BK && ((uintptr_t)sx & 15) == 0 &&
                       (B == 1 || sx_ws % 4 == 0) && !getenv("BNH_PROTO_WINDOW");
  if (batched) {
    static int ncu = 0;
    if (!ncu) {
      int dev = 0;
      BNH_HIP(hipGetDevice(&dev));
      BNH_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
    }
    const int n_mt = (int)bnh_ceil_div((long long)B * 64, PG_TM), n_nt = W->Npt / PG_TN;
    int grid = ncu / 8 * 8;  // one block per CU
    if (grid < 8) grid = 8;
    static const bool four = getenv("BNH_PROTO_4W") != nullptr;  // the 4-wave form, for comparison
    if (four)
      hipLaunchKernelGGL(k_proto_gemm64, dim3((unsigned)grid), dim3(256), 0, bnh_stream(stream), qa, B == 1 ? 0 : qa_ws,
                         sx, B == 1 ? 0 : sx_ws, B, W->Kp, W->w, W->sw, W->Np, n_mt, n_nt, colmax, B == 1 ? 0 : cm_ws);
    else
      hipLaunchKernelGGL(k_proto_gemm_pp, dim3((unsigned)grid), dim3(512), 0, bnh_stream(stream), qa, B == 1 ? 0 : qa_ws,
                         sx, B == 1 ? 0 : sx_ws, B, W->Kp, W->w, W->sw, W->Np, n_mt, n_nt, colmax, B == 1 ? 0 : cm_ws);
    BNH_HIP(hipGetLastError());
    return 0;
  }
  BNH_REQ(B <= 65535 * 1024);
  dim3 grid((unsigned)B, (unsigned)(W->Npt / 256));
  hipLaunchKernelGGL(k_proto_colmax, grid, dim3(256), 0, bnh_stream(stream), qa, qa_ws, W->Kp, sx, sx_ws, P, W->w, W->sw,
                     W->Np, colmax, cm_ws);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_proto_logits(const float *colmax, long long cm_ws, const float *clsw, const float *clsb, int nc, int ppc,
                     float *logits, long long lg_ws, int B, int *win_fail, int fail_code, void *stream) {
  BNH_REQ(colmax && clsw && clsb && logits && nc > 0 && ppc > 0 && B > 0);
  BNH_REQ(B == 1 || (cm_ws >= (long long)nc * ppc && lg_ws >= nc));
  const long long n = (long long)nc * B;
  hipLaunchKernelGGL(k_proto_logits, dim3((unsigned)bnh_ceil_div(n, 256)), dim3(256), 0, bnh_stream(stream), colmax,
                     cm_ws, clsw, clsb, nc, ppc, logits, lg_ws, B, win_fail, fail_code);
  BNH_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
