// fp16 Winograd F(2x2, 3x3) convolution, stride 1, 'same' (pad 1), on gfx950 fp16 MFMA (the Winograd / fp16 GEMM
// path of libbnneon: src/wino_s0.c's transform structure, src/wino.c's tiling), one fused kernel:
//
//   V = B^T d B   per 4x4 input tile and input channel   (fp16 adds in wino_s0.c's order, in_tf :80-97)
//   M_p = V_p U_p per position p = 0..15                  (fp16 MFMA, fp32 accumulation over the input channels)
//   y = A^T M A + b, activation, + residual               (fp32, one rounding to fp16 at the end)
//
// with U = G g G^T computed once at load in fp32 and rounded to fp16 (wino_s0_pack, :40-64). Coefficients:
// B^T = [[1,0,-1,0],[0,1,1,0],[0,-1,1,0],[0,1,0,-1]], G = [[1,0,0],[.5,.5,.5],[.5,-.5,.5],[0,0,1]],
// A^T = [[1,1,1,0],[0,1,-1,-1]].
//
// Work split: a block owns one window's strip of 32 output columns (16 tiles across) and walks its tile rows
// (steps) in a software pipeline of two wave groups, one block barrier per phase:
//   * producers (NCO waves), in phase P: the input transform of step P from a 6-row LDS ring of input rows into
//     V[P & 1] [16 positions][16 tiles][Cp]; the ring rows of step P + 1 written from registers, and the loads of
//     the rows after issued (coalesced 8-byte loads of whole row segments: each input row is read once per strip);
//     and the epilogue of step P - 2 from the fp32 LDS output tile Os[P & 1] (bias, activation, rounding to fp16,
//     residual) stored as channel-contiguous 16-byte rows;
//   * consumers (NCO waves, each owning 16 output channels and their U fragments for all 16 positions and input
//     channels in registers for the whole strip), in phase P: the 16 x Cp/32 MFMAs of step P - 1 (A = V rows of 16
//     tiles, B = its U) and the output transform in registers (a lane holds all 16 positions of 4 tiles for one
//     channel) into Os[(P - 1) & 1] (fp32).
// The two groups share each SIMD, so the transforms, matrix products and memory traffic of neighbouring steps
// overlap. The epilogue's SiLU is y / (1 + 2^(-y log2 e)) on the hardware exp2 and reciprocal (about 1 ulp of fp32
// each), far inside the fp16 tolerance of this path.
#include <math.h>
#include <string.h>

#include <type_traits>

#include "bnh_internal.h"
#include "bnh_num.h"
#include "bnh_f16.h"

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

struct bnh_wino16 {
  int C, K, Cp, Kp;  // Cp = C rounded up to 32 (the MFMA k step), Kp = K rounded up to 16
  uint16_t *U;       // [16][Kp][Cp] fp16, zero past C and K
  float *b;          // [Kp]
};

#define WT_TILES 16  // tiles per step (the MFMA row dimension)
#define WT_COLS 34   // input columns of a strip: 2 x 16 + 2

BNH_DEV float wino_silu(float y) {
  const float t = __builtin_amdgcn_exp2f(-1.44269504f * y);
  const float s = y * __builtin_amdgcn_rcpf(1.0f + t);
  return y == -INFINITY ? -0.0f : s;
}

template <int NCO, int NCH, int ACT>  // NCO waves of 16 output channels, NCH = Cp / 32 MFMA k steps, ACT 0/1/2
__global__ __launch_bounds__(128 * NCO) void k_wino_f16(const uint16_t *__restrict__ x, long long x_ws, int H, int W,
                                                        int C, int ldx, const uint16_t *__restrict__ U,
                                                        const float *__restrict__ bias, int K,
                                                        uint16_t *__restrict__ out, long long o_ws, int ldo, int opad,
                                                        const uint16_t *__restrict__ res, long long r_ws, int ldr,
                                                        int rpad, int strips, int vec) {
  constexpr int CP = 32 * NCH, KP = 16 * NCO, NA = 64 * NCO, RING = 6;
  // padded strides: ring pixel (halves; two pixels apart = 32 banks, so a wave's in-transform reads of two tiles
  // share no bank), V tile (halves; the 16 tiles of an MFMA operand read in distinct banks), output pixel (floats)
  constexpr int XS = CP == 64 ? 96 : 48, VS = CP + 8, OS = KP + 4;
  constexpr int VSZ = 16 * WT_TILES * VS, OSZ = 2 * 2 * WT_TILES * OS;
  constexpr int PRE = (2 * WT_COLS * (CP / 4) + NA - 1) / NA;   // prefetch slots per producer (8-byte chunks)
  constexpr int SV = (2 * 2 * WT_TILES * KP / 8 + NA - 1) / NA;  // 16-byte output items per producer
  __shared__ __attribute__((aligned(16))) _Float16 Xs[RING * WT_COLS * XS];
  __shared__ __attribute__((aligned(16))) _Float16 V[2 * VSZ];
  __shared__ __attribute__((aligned(16))) float Os[2 * OSZ];
  __shared__ __attribute__((aligned(16))) float Bs[KP];  // the bias
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool prod = tid < NA;
  const int win = blockIdx.x / strips, strip = blockIdx.x % strips;
  const int T = W / 2, tx0 = strip * WT_TILES, Wp = W + 2, c4 = C / 4, NS = H / 2;
  const int npx = 2 * (T - tx0 < WT_TILES ? T - tx0 : WT_TILES);  // output columns of the strip
  // ---- producer state: the window's haloed input as a buffer (columns past the image read zeros or the next row;
  // tiles past T are never stored); per prefetch slot: its row (-1: none), byte offset from the first row's strip
  // start and LDS offset within a ring row; per 16-byte output item: Os offset (-1: none) and element offsets of the
  // output and residual from output row 2 step's start
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(x + win * x_ws), 0, (int)((long long)(H + 2) * Wp * ldx * 2), 0x00020000);
  uint2 pre[PRE];
  int pr[PRE], pg[PRE], pl[PRE];
#pragma unroll
  for (int j = 0; j < PRE; j++) {
    const int i = tid + NA * j, r = i / (WT_COLS * c4), rem = i - r * (WT_COLS * c4), px = rem / c4, g = rem - px * c4;
    pr[j] = prod && r < 2 ? r : -1;
    pg[j] = ((r * Wp + 2 * tx0 + px) * ldx + 4 * g) * 2;
    pl[j] = px * XS + 4 * g;
  }
  int so[SV], sg[SV], sr[SV];
  {
    const int k8 = vec ? K / 8 : 1;
#pragma unroll
    for (int j = 0; j < SV; j++) {
      const int it = tid + NA * j, i = it / (npx * k8), rem = it - i * (npx * k8), px = rem / k8, ch = 8 * (rem - px * k8);
      const int ox = 2 * tx0 + px;
      so[j] = prod && vec && it < 2 * npx * k8 ? (i * 2 * WT_TILES + px) * OS + ch : -1;
      sg[j] = ((i + opad) * (W + 2 * opad) + ox + opad) * ldo + ch;
      sr[j] = ((i + rpad) * (W + 2 * rpad) + ox + rpad) * ldr + ch;
    }
  }
  const long long orowb = (long long)(W + 2 * opad) * ldo, rrowb = (long long)(W + 2 * rpad) * ldr;
  const int rowb = Wp * ldx * 2;
  auto fetch = [&](uint2 (&dst)[PRE], int r0) {  // rows r0, r0 + 1 -> registers (the whole offset range-checked)
#pragma unroll
    for (int j = 0; j < PRE; j++) {
      dst[j] = make_uint2(0u, 0u);
      if (pr[j] >= 0) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(xr, pg[j] + r0 * rowb, 0, 0);
        dst[j] = make_uint2(v[0], v[1]);
      }
    }
  };
  auto commit = [&](int r0) {  // the prefetched rows r0, r0 + 1 into their ring slots
#pragma unroll
    for (int j = 0; j < PRE; j++)
      if (pr[j] >= 0) *(uint2 *)(Xs + ((r0 + pr[j]) % RING) * WT_COLS * XS + pl[j]) = pre[j];
  };
  // ---- consumer state: this wave's U fragments (position p, k step c -> channels co = 16 (wave - NCO) + (lane & 15),
  // input channels 32 c + 8 (lane >> 4) .. + 7)
  const int co = 16 * (wave - NCO) + (lane & 15);
  v8h u[16][NCH];
  if (!prod) {
#pragma unroll
    for (int p = 0; p < 16; p++)
#pragma unroll
      for (int c = 0; c < NCH; c++)
        u[p][c] = *(const v8h *)(U + ((long long)(p * KP + co)) * CP + 32 * c + 8 * (lane >> 4));
  }
  if (prod) {  // the bias; rows 0..3 of step 0, and the loads of rows 4, 5
    for (int i = tid; i < KP; i += NA) Bs[i] = bias[i];
    fetch(pre, 0);
    commit(0);
    fetch(pre, 2);
    commit(2);
    if (NS > 1) fetch(pre, 4);
  }
  __syncthreads();
  for (int P = 0; P <= NS + 1; P++) {
    if (prod) {
      // ---- V = B^T d B for the 16 tiles of step P (fp16, wino_s0.c in_tf order); channel quads past C are zero
      if (P < NS) {
        _Float16 *Vb = V + (P & 1) * VSZ;
        for (int it = tid; it < WT_TILES * (CP / 4); it += NA) {
          const int g = it % (CP / 4), t = it / (CP / 4);
          v4h vv[16];
          if (g < c4) {
            v4h dd[4][4];
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
              for (int cc = 0; cc < 4; cc++)
                dd[r][cc] = *(const v4h *)(Xs + (((2 * P + r) % RING) * WT_COLS + 2 * t + cc) * XS + 4 * g);
            v4h tt[4][4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
              tt[0][j] = dd[0][j] - dd[2][j];
              tt[1][j] = dd[1][j] + dd[2][j];
              tt[2][j] = dd[2][j] - dd[1][j];
              tt[3][j] = dd[1][j] - dd[3][j];
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
              vv[4 * i + 0] = tt[i][0] - tt[i][2];
              vv[4 * i + 1] = tt[i][1] + tt[i][2];
              vv[4 * i + 2] = tt[i][2] - tt[i][1];
              vv[4 * i + 3] = tt[i][1] - tt[i][3];
            }
          } else {
#pragma unroll
            for (int p = 0; p < 16; p++) vv[p] = (v4h){};
          }
#pragma unroll
          for (int p = 0; p < 16; p++) *(v4h *)(Vb + (p * WT_TILES + t) * VS + 4 * g) = vv[p];
        }
        if (P + 1 < NS) commit(2 * P + 4);  // rows of step P + 1, read after this phase's barrier
        if (P + 2 < NS) fetch(pre, 2 * P + 6);
      }
      // ---- step P - 2's two output rows: + b, activation, fp16 (residual added in fp16 after the rounding)
      if (P >= 2) {
        const int ty = P - 2;
        const float *Ob = Os + (P & 1) * OSZ;
        auto epi = [&](float y, float b) {
          y = y + b;
          if (ACT == 1) y = wino_silu(y);
          else if (ACT == 2) y = bnh_relu_f32(y);
          return f2h(y);
        };
        if (vec) {  // 8 channels per item: 16-byte stores
#pragma unroll
          for (int j = 0; j < SV; j++) {
            if (so[j] < 0) continue;
            const float4 y0 = *(const float4 *)(Ob + so[j]), y1 = *(const float4 *)(Ob + so[j] + 4);
            const int ch = so[j] % OS;
            const float4 b0 = *(const float4 *)(Bs + ch), b1 = *(const float4 *)(Bs + ch + 4);
            auto pk = [&](float a, float b, float ba, float bb) {
              const h2 v = (h2){epi(a, ba), epi(b, bb)};
              return __builtin_bit_cast(uint32_t, v);
            };
            uint4 v = make_uint4(pk(y0.x, y0.y, b0.x, b0.y), pk(y0.z, y0.w, b0.z, b0.w), pk(y1.x, y1.y, b1.x, b1.y),
                                 pk(y1.z, y1.w, b1.z, b1.w));
            if (res) {
              const uint4 rv = *(const uint4 *)(res + win * r_ws + (long long)(2 * ty) * rrowb + sr[j]);
              v = make_uint4(__builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v.x) + __builtin_bit_cast(h2, rv.x)),
                             __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v.y) + __builtin_bit_cast(h2, rv.y)),
                             __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v.z) + __builtin_bit_cast(h2, rv.z)),
                             __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v.w) + __builtin_bit_cast(h2, rv.w)));
            }
            *(uint4 *)(out + win * o_ws + (long long)(2 * ty) * orowb + sg[j]) = v;
          }
        } else {
          for (int it = tid; it < 2 * npx * K; it += NA) {
            const int i = it / (npx * K), rem = it - i * (npx * K), px = rem / K, ch = rem - px * K;
            const int oy = 2 * ty + i, ox = 2 * tx0 + px;
            h16 v = epi(Ob[(i * 2 * WT_TILES + px) * OS + ch], Bs[ch]);
            if (res) {
              const long long rrow = rpad ? (long long)(oy + rpad) * (W + 2 * rpad) + ox + rpad : (long long)oy * W + ox;
              v = v + hfrom(res[win * r_ws + rrow * ldr + ch]);
            }
            const long long orow = opad ? (long long)(oy + opad) * (W + 2 * opad) + ox + opad : (long long)oy * W + ox;
            out[win * o_ws + orow * ldo + ch] = hbits(v);
          }
        }
      }
    } else if (P >= 1 && P <= NS) {
      // ---- M_p = V_p U_p for step P - 1: lane rows = tiles 4 (lane >> 4) + r, column = channel co
      const _Float16 *Vb = V + ((P - 1) & 1) * VSZ;
      v4f acc[16];
#pragma unroll
      for (int p = 0; p < 16; p++) {
        acc[p] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NCH; c++) {
          const v8h a = *(const v8h *)(Vb + (p * WT_TILES + (lane & 15)) * VS + 32 * c + 8 * (lane >> 4));
          acc[p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, u[p][c], acc[p], 0, 0, 0);
        }
      }
      // ---- y = A^T M A per tile (fp32): 2 x 2 outputs of channel co into the output tile
      float *Ob = Os + ((P - 1) & 1) * OSZ;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int t = 4 * (lane >> 4) + r;
        float s[2][4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          s[0][j] = (acc[j][r] + acc[4 + j][r]) + acc[8 + j][r];
          s[1][j] = (acc[4 + j][r] - acc[8 + j][r]) - acc[12 + j][r];
        }
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
          for (int jx = 0; jx < 2; jx++) {
            Ob[(i * 2 * WT_TILES + 2 * t + jx) * OS + co] =
                jx == 0 ? (s[i][0] + s[i][1]) + s[i][2] : (s[i][1] - s[i][2]) - s[i][3];
          }
      }
    }
    __syncthreads();
  }
}

// Version 2 (position-row waves; channel counts that are multiples of 8, 4-channel aligned outputs). The block is
// 4 waves and owns the same strip of 16 tiles as above; wave i owns row i of the 16 Winograd positions
// (p = 4 i + j) for every output channel, and computes the V operands of its row itself, in registers, straight from
// the ring of input rows: row i of B^T d combines two input rows (d0 - d2, d1 + d2, d2 - d1, d1 - d3), then the four
// column combinations give V[i][0..3] in the order of the form above (same fp16 adds, same bits). So V is never
// written to LDS or read back once per consumer wave; the wave's U fragments (its 4 positions x every channel pair,
// 128 VGPRs at 64 x 64) stay in registers for the strip. Each 16-channel block's four position products are summed
// over the columns in registers (M A: two values per tile row; row 1's position-1 product starts from the bias, which
// every output takes exactly once through row 1) and exchanged through LDS as S[i][tile][jx][co]; after a barrier
// every thread takes a tile and 4 output channels and finishes A^T (M A) over the rows, the activation, fp16 and the
// residual, with 8-byte stores. Two barriers per step (S written / S read); 62 KB of LDS at 64 x 64, so two blocks
// share a CU and one block's epilogue runs beside the other's products. The fp32 output transform sums the columns
// first (the form above sums the rows first) and carries the bias inside it: the same bound, other fp32 roundings.

// wino_silu with the DX9 multiply (v_mul_legacy_f32: 0 x anything = +0), so that y = -inf, whose reciprocal factor
// is 0, gives +0 without a compare and select; every other input gives wino_silu's value (NaN stays NaN). The
// reciprocal and the multiply are one asm block with the wait state a VALU read of a transcendental result needs
// (the compiler inserts none for registers an asm statement reads).
BNH_DEV float wino_silu_l(float y) {
  const float a = 1.0f + __builtin_amdgcn_exp2f(-1.44269504f * y);
  float d, r;
  asm("v_rcp_f32 %1, %3\n\ts_nop 0\n\tv_mul_legacy_f32 %0, %2, %1" : "=v"(d), "=&v"(r) : "v"(y), "v"(a));
  return d;
}

// Eight fp16 channels as four pairs. The transforms below run on the pairs so that every add and subtract is one
// v_pk_add_f16 (the compiler turns 8-wide fp16 subtractions into scalar v_sub_f16 pairs and repacks them, 3
// instructions per pair).
struct H8 {
  h2 h[4];
};
BNH_DEV H8 h8_ld(const _Float16 *p) {
  H8 r;
  __builtin_memcpy(&r, p, 16);
  return r;
}
BNH_DEV H8 h8_add(H8 a, H8 b) {
  H8 r;
#pragma unroll
  for (int k = 0; k < 4; k++) r.h[k] = a.h[k] + b.h[k];
  return r;
}
BNH_DEV H8 h8_sub(H8 a, H8 b) {
  H8 r;
#pragma unroll
  for (int k = 0; k < 4; k++) r.h[k] = a.h[k] - b.h[k];
  return r;
}
BNH_DEV v8h h8_v(H8 a) {
  v8h o;
  __builtin_memcpy(&o, &a, 16);
  return o;
}

template <int NCH, int NCB, int ACT>  // NCH = Cp / 32 MFMA k steps, NCB = Kp / 16 output channel blocks
__global__ __launch_bounds__(256, 2) void k_wino_f16r(const uint16_t *__restrict__ x, long long x_ws, int H, int W,
                                                      int C, int ldx, const uint16_t *__restrict__ U,
                                                      const float *__restrict__ bias, int K,
                                                      uint16_t *__restrict__ out, long long o_ws, int ldo, int opad,
                                                      const uint16_t *__restrict__ res, long long r_ws, int ldr,
                                                      int rpad, int strips) {
  constexpr int CP = 32 * NCH, KP = 16 * NCB, RING = 6;
  constexpr int XS = CP + 8;                 // ring pixel stride (halves)
  constexpr int XR = WT_COLS * XS;           // ring row stride (halves)
  constexpr int SS = 2 * KP + 4;             // S tile stride (floats): a write's 4 tile groups in distinct banks
  constexpr int NQ = CP / 8;                 // 16-byte chunks of a pixel
  constexpr int NLD = 2 * WT_COLS * NQ;      // chunks of two ring rows
  constexpr int PRE = (NLD + 255) / 256;     // prefetch slots per thread
  __shared__ __attribute__((aligned(16))) _Float16 Xs[RING * XR];
  __shared__ __attribute__((aligned(16))) float Ss[4 * WT_TILES * SS];
  __shared__ __attribute__((aligned(16))) float Bs[KP];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wi = __builtin_amdgcn_readfirstlane(tid >> 6);  // this wave's row of positions
  const int win = blockIdx.x / strips, strip = blockIdx.x % strips;
  const int T = W / 2, tx0 = strip * WT_TILES, Wp = W + 2, NS = H / 2, c8 = C / 8;
  const int ntl = T - tx0 < WT_TILES ? T - tx0 : WT_TILES;  // tiles of this strip that are stored
  // the window's haloed input as one buffer (columns past the image read the next row or zeros; tiles past T are
  // never stored)
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(x + win * x_ws), 0, (int)((long long)(H + 2) * Wp * ldx * 2), 0x00020000);
  const int rowb = Wp * ldx * 2;
  // prefetch slot j: chunk q of pixel px of ring row r (0 / 1 of the pair); -1 past the pair or past C
  int pgo[PRE], plo[PRE], prr[PRE];
#pragma unroll
  for (int j = 0; j < PRE; j++) {
    const int it = tid + 256 * j, r = it / (WT_COLS * NQ), rem = it - r * (WT_COLS * NQ), px = rem / NQ,
              q = rem - px * NQ;
    const bool ok = it < NLD && q < c8;
    prr[j] = ok ? r : -1;
    pgo[j] = ((r * Wp + 2 * tx0 + px) * ldx + 8 * q) * 2;
    plo[j] = (r * XR + px * XS + 8 * q) * 2;  // bytes from the pair's first ring row
  }
  v4i pre[PRE];
  auto fetch = [&](int r0) {
#pragma unroll
    for (int j = 0; j < PRE; j++)
      pre[j] = prr[j] >= 0 ? __builtin_amdgcn_raw_buffer_load_b128(xr, pgo[j] + r0 * rowb, 0, 0) : (v4i){0, 0, 0, 0};
  };
  auto commit = [&](int slot0) {  // the pair into ring rows slot0, slot0 + 1 (slot0 even, so never wrapping)
    char *xb = (char *)(Xs + slot0 * XR);
#pragma unroll
    for (int j = 0; j < PRE; j++)
      if (prr[j] >= 0) *(v4i *)(xb + plo[j]) = pre[j];
  };
  // this wave's U fragments: position p = 4 wi + j, k step c, channel block cb -> output channel
  // 16 cb + (lane & 15), input channels 32 c + 8 (lane >> 4) .. + 7
  v8h u[4][NCH][NCB];
#pragma unroll
  for (int j = 0; j < 4; j++)
#pragma unroll
    for (int c = 0; c < NCH; c++)
#pragma unroll
      for (int cb = 0; cb < NCB; cb++)
        u[j][c][cb] = *(const v8h *)(U + ((long long)((4 * wi + j) * KP + 16 * cb + (lane & 15))) * CP + 32 * c +
                                     8 * (lane >> 4));
  if (c8 < NQ)  // channels past C read as zeros: no load ever writes them
    for (int i = tid; i < RING * XR / 8; i += 256) ((v4i *)Xs)[i] = (v4i){0, 0, 0, 0};
  for (int i = tid; i < KP; i += 256) Bs[i] = i < K ? bias[i] : 0.f;
  __syncthreads();
  fetch(0);
  commit(0);
  fetch(2);
  commit(2);
  if (NS > 1) fetch(4);
  // the output and residual of the window as buffers: 32-bit byte offsets, a lane part and a scalar row part
  const __amdgpu_buffer_rsrc_t orr = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(out + win * o_ws), 0, (int)((long long)(H + 2 * opad) * (W + 2 * opad) * ldo * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rrr = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(res ? res + win * r_ws : out), 0, res ? (int)((long long)(H + 2 * rpad) * (W + 2 * rpad) * ldr * 2) : 0,
      0x00020000);
  __syncthreads();
  // row i of B^T d: d[ra] - d[rb] (i = 0, 2, 3) or d[ra] + d[rb] (i = 1)
  const int ra = wi == 0 ? 0 : wi == 2 ? 2 : 1, rb = wi == 0 ? 2 : wi == 3 ? 3 : wi == 1 ? 2 : 1;
  const int xl = (2 * (lane & 15)) * XS + 8 * (lane >> 4);  // this lane's tile's first column, its channel group
  // epilogue item: tile et, output channels 4 eq .. 4 eq + 3
  const int et = tid >> 4, eq = tid & 15;
  const bool eon = et < ntl && 4 * eq < K;
  const int orow = (W + 2 * opad) * ldo * 2, rrow = (W + 2 * rpad) * ldr * 2;  // bytes per row
  const int ol = ((opad * (W + 2 * opad) + 2 * (tx0 + et) + opad) * ldo + 4 * eq) * 2;
  const int rl = ((rpad * (W + 2 * rpad) + 2 * (tx0 + et) + rpad) * ldr + 4 * eq) * 2;
  float binit[NCB];  // row 1's position-1 sums start from the bias of the lane's output channel in each block
#pragma unroll
  for (int cb = 0; cb < NCB; cb++) binit[cb] = wi == 1 ? Bs[16 * cb + (lane & 15)] : 0.f;
  // the step loop, compiled once for row 1 (an add of the two input rows) and once for the others (a subtraction),
  // so that no wave branches per instruction on its row
  auto steps = [&](auto add_rows) {
  constexpr bool ADD = decltype(add_rows)::value;
  int base = 0;  // ring row of the step's first input row
  for (int s = 0; s < NS; s++) {
    // the rows of step s + 1 (loaded during step s - 1) into the ring slots step s - 1 read last
    if (s + 1 < NS) commit(base == 0 ? 4 : base - 2);
    if (s + 2 < NS) fetch(2 * s + 6);
    // ---- V operands of row wi for the 16 tiles, every k step
    v8h vv[4][NCH];
    const _Float16 *xa = Xs + ((base + ra) % RING) * XR + xl, *xb = Xs + ((base + rb) % RING) * XR + xl;
#pragma unroll
    for (int c = 0; c < NCH; c++) {
      H8 tt[4];
#pragma unroll
      for (int cc = 0; cc < 4; cc++) {
        const H8 da = h8_ld(xa + cc * XS + 32 * c), db = h8_ld(xb + cc * XS + 32 * c);
        tt[cc] = ADD ? h8_add(da, db) : h8_sub(da, db);
      }
      vv[0][c] = h8_v(h8_sub(tt[0], tt[2]));
      vv[1][c] = h8_v(h8_add(tt[1], tt[2]));
      vv[2][c] = h8_v(h8_sub(tt[2], tt[1]));
      vv[3][c] = h8_v(h8_sub(tt[1], tt[3]));
      __builtin_amdgcn_sched_barrier(0);  // one k step's input chunks live at a time (VGPRs: U holds 128)
    }
    // ---- per channel block: the four position products (row 1's position 1 starts from the bias, which every
    // output takes once through it), then M A over the columns into S
    float *sw = Ss + wi * WT_TILES * SS + (lane & 15);
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
      v4f m[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        m[j] = j == 1 ? (v4f){binit[cb], binit[cb], binit[cb], binit[cb]} : (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NCH; c++) m[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv[j][c], u[j][c][cb], m[j], 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int tile = 4 * (lane >> 4) + r;
        float *d = sw + tile * SS + 16 * cb;
        d[0] = (m[0][r] + m[1][r]) + m[2][r];
        d[KP] = (m[1][r] - m[2][r]) - m[3][r];
      }
    }
    __syncthreads();
    // ---- y = A^T (M A) + b, activation, fp16, residual: tile et, channels 4 eq .. + 3, both output rows and columns
    if (eon) {
      float4 sv[4][2];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jx = 0; jx < 2; jx++) sv[i][jx] = *(const float4 *)(Ss + (i * WT_TILES + et) * SS + jx * KP + 4 * eq);
      auto epi = [&](float y) {  // the bias is in S[1]
        if (ACT == 1) y = wino_silu_l(y);
        else if (ACT == 2) y = bnh_relu_f32(y);
        return f2h(y);
      };
#pragma unroll
      for (int iy = 0; iy < 2; iy++)
#pragma unroll
        for (int jx = 0; jx < 2; jx++) {
          const float4 a = sv[0][jx], b = sv[1][jx], c = sv[2][jx], e = sv[3][jx];
          float4 y;
          if (iy == 0) y = make_float4((a.x + b.x) + c.x, (a.y + b.y) + c.y, (a.z + b.z) + c.z, (a.w + b.w) + c.w);
          else y = make_float4((b.x - c.x) - e.x, (b.y - c.y) - e.y, (b.z - c.z) - e.z, (b.w - c.w) - e.w);
          h2 lo = (h2){epi(y.x), epi(y.y)}, hi = (h2){epi(y.z), epi(y.w)};
          if (res) {
            const v2u rv = __builtin_amdgcn_raw_buffer_load_b64(rrr, rl, (2 * s + iy) * rrow + jx * ldr * 2, 0);
            // the words as scalars first: hipcc miscompiles __builtin_bit_cast of an ext_vector element (it reads
            // element 0 for every index)
            const uint32_t r0 = rv.x, r1 = rv.y;
            lo = lo + __builtin_bit_cast(h2, r0);
            hi = hi + __builtin_bit_cast(h2, r1);
          }
          __builtin_amdgcn_raw_buffer_store_b64(
              (v2u){__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)}, orr, ol,
              (2 * s + iy) * orow + jx * ldo * 2, 0);
        }
    }
    __syncthreads();
    base = base + 2 == RING ? 0 : base + 2;
  }
  };
  if (wi == 1) steps(std::true_type{});
  else steps(std::false_type{});
}

__global__ void k_zero_halo16(uint16_t *__restrict__ out, long long ws, int H, int W, int C, int h, long long total) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int Wp = W + 2 * h;
  const long long per = (long long)(H + 2 * h) * Wp * C;
  const int w = (int)(i / per);
  const long long el = i % per, px = el / C;
  const int y = (int)(px / Wp), xx = (int)(px % Wp);
  if (y >= h && y < H + h && xx >= h && xx < W + h) return;
  out[w * ws + el] = 0;
}

extern "C" {

bnh_wino16 *bnh_wino16_new(int C, int K, const float *w, const float *bias) {
  if (C <= 0 || K <= 0 || C % 4 || C > 64 || K > 64 || !w) {
    bnh_fail("bnh_wino16_new: C %d K %d: expected C %% 4 == 0, C <= 64, K <= 64 and the weights", C, K);
    return nullptr;
  }
  const int Cp = (int)bnh_round_up(C, 32), Kp = (int)bnh_round_up(K, 16);
  uint16_t *hu = (uint16_t *)calloc((size_t)16 * Kp * Cp, 2);
  float *hb = (float *)calloc(Kp, 4);
  bnh_wino16 *P = (bnh_wino16 *)calloc(1, sizeof *P);
  if (!hu || !hb || !P) {
    free(hu); free(hb); free(P);
    bnh_fail("bnh_wino16_new: out of host memory");
    return nullptr;
  }
  static const float G[4][3] = {{1, 0, 0}, {.5f, .5f, .5f}, {.5f, -.5f, .5f}, {0, 0, 1}};
  for (int o = 0; o < K; o++) {
    hb[o] = bias ? bias[o] : 0.f;
    for (int ci = 0; ci < C; ci++) {  // w OHWI [K][3][3][C] fp32; U = G g G^T in fp32, rounded to fp16
      float g[3][3], t[4][3];
      for (int ky = 0; ky < 3; ky++)
        for (int kx = 0; kx < 3; kx++) g[ky][kx] = w[((o * 3 + ky) * 3 + kx) * C + ci];
      for (int i = 0; i < 4; i++)
        for (int kx = 0; kx < 3; kx++) t[i][kx] = G[i][0] * g[0][kx] + G[i][1] * g[1][kx] + G[i][2] * g[2][kx];
      for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) {
          const float uv = t[i][0] * G[j][0] + t[i][1] * G[j][1] + t[i][2] * G[j][2];
          const _Float16 hv = (_Float16)uv;
          memcpy(&hu[((size_t)(i * 4 + j) * Kp + o) * Cp + ci], &hv, 2);
        }
    }
  }
  P->C = C; P->K = K; P->Cp = Cp; P->Kp = Kp;
  bool ok = (P->U = (uint16_t *)bnh_malloc((size_t)16 * Kp * Cp * 2)) && (P->b = (float *)bnh_malloc(4 * (size_t)Kp)) &&
            !bnh_memcpy_h2d(P->U, hu, (size_t)16 * Kp * Cp * 2) && !bnh_memcpy_h2d(P->b, hb, 4 * (size_t)Kp);
  free(hu); free(hb);
  if (!ok) { bnh_wino16_free(P); return nullptr; }
  return P;
}

void bnh_wino16_free(bnh_wino16 *P) {
  if (!P) return;
  if (P->U) (void)hipFree(P->U);
  if (P->b) (void)hipFree(P->b);
  free(P);
}

int bnh_wino_f16(const uint16_t *x, long long x_ws, int H, int W, int ldx, const bnh_wino16 *P, int act, uint16_t *out,
                 long long o_ws, int ldo, int opad, const uint16_t *res, long long r_ws, int ldr, int rpad, int B,
                 void *stream) {
  BNH_REQ(x && P && out && H > 0 && W > 0 && H % 2 == 0 && W % 2 == 0 && B > 0);
  BNH_REQ(ldx >= P->C && ldx % 4 == 0 && ldo >= P->K && (opad == 0 || opad == 1) && act >= 0 && act <= 2);
  BNH_REQ(((uintptr_t)x & 7) == 0 && (B == 1 || x_ws % 4 == 0));
  BNH_REQ(!res || (ldr >= P->K && (rpad == 0 || rpad == 1)));
  BNH_REQ(!res || B == 1 || r_ws >= (long long)(H + 2 * rpad) * (W + 2 * rpad) * ldr);
  BNH_REQ(B == 1 || (x_ws >= (long long)(H + 2) * (W + 2) * ldx && o_ws >= (long long)(H + 2 * opad) * (W + 2 * opad) * ldo));
  hipStream_t st = bnh_stream(stream);
  if (opad) {
    const long long per = (long long)(H + 2) * (W + 2) * ldo, total = per * B;
    hipLaunchKernelGGL(k_zero_halo16, dim3((unsigned)bnh_ceil_div(total, 256)), dim3(256), 0, st, out,
                       B == 1 ? per : o_ws, H, W, ldo, 1, total);
    BNH_HIP(hipGetLastError());
  }
  const int strips = (int)bnh_ceil_div(W / 2, WT_TILES);
  const dim3 grid((unsigned)((long long)strips * B));
  const int nco = P->Kp / 16, nch = P->Cp / 32;
  // version 2 (position-row waves) when 16-byte input chunks and 8-byte output quads are aligned;
  // BNH_WINO_FORM=1 keeps version 1, for comparison
  static const bool v1 = [] {
    const char *e = getenv("BNH_WINO_FORM");
    return e && e[0] == '1';
  }();
  const bool r_ok = P->C % 8 == 0 && ldx % 8 == 0 && ((uintptr_t)x & 15) == 0 && (B == 1 || x_ws % 8 == 0) &&
                    P->K % 4 == 0 && ldo % 4 == 0 && ((uintptr_t)out & 7) == 0 && (B == 1 || o_ws % 4 == 0) &&
                    (!res || (ldr % 4 == 0 && ((uintptr_t)res & 7) == 0 && (B == 1 || r_ws % 4 == 0)));
  if (r_ok && !v1) {
#define WINOR_A(NCH, NCB, ACT)                                                                                         \
  hipLaunchKernelGGL((k_wino_f16r<NCH, NCB, ACT>), grid, dim3(256), 0, st, x, x_ws, H, W, P->C, ldx, P->U, P->b, P->K, \
                     out, o_ws, ldo, opad, res, r_ws, ldr, rpad, strips)
#define WINOR(NCH, NCB)                                                                                                \
  do {                                                                                                                 \
    if (act == 1) WINOR_A(NCH, NCB, 1);                                                                                \
    else if (act == 2) WINOR_A(NCH, NCB, 2);                                                                           \
    else WINOR_A(NCH, NCB, 0);                                                                                         \
  } while (0)
    if (nch == 1) {
      if (nco == 1) WINOR(1, 1); else if (nco == 2) WINOR(1, 2); else if (nco == 3) WINOR(1, 3); else WINOR(1, 4);
    } else {
      if (nco == 1) WINOR(2, 1); else if (nco == 2) WINOR(2, 2); else if (nco == 3) WINOR(2, 3); else WINOR(2, 4);
    }
#undef WINOR
#undef WINOR_A
    BNH_HIP(hipGetLastError());
    return 0;
  }
  // a window's input is one buffer resource; per-window element offsets of the output and residual fit 32 bits
  BNH_REQ((long long)(H + 2) * (W + 2) * ldx * 2 < (1LL << 31));
  BNH_REQ((long long)(H + 2 * opad) * (W + 2 * opad) * ldo < (1LL << 31));
  BNH_REQ(!res || (long long)(H + 2 * rpad) * (W + 2 * rpad) * ldr < (1LL << 31));
  // 16-byte output rows when every 8-channel group is aligned
  const int vec = P->K % 8 == 0 && ldo % 8 == 0 && ((uintptr_t)out & 15) == 0 && (B == 1 || o_ws % 8 == 0) &&
                  (!res || (ldr % 8 == 0 && ((uintptr_t)res & 15) == 0 && (B == 1 || r_ws % 8 == 0)));
#define WINO_LAUNCH(NCO, NCH)                                                                                          \
  do {                                                                                                                 \
    if (act == 1) WINO_LAUNCH_A(NCO, NCH, 1);                                                                          \
    else if (act == 2) WINO_LAUNCH_A(NCO, NCH, 2);                                                                     \
    else WINO_LAUNCH_A(NCO, NCH, 0);                                                                                   \
  } while (0)
#define WINO_LAUNCH_A(NCO, NCH, ACT)                                                                                   \
  hipLaunchKernelGGL((k_wino_f16<NCO, NCH, ACT>), grid, dim3(128 * NCO), 0, st, x, x_ws, H, W, P->C, ldx, P->U, P->b,   \
                     P->K, out, o_ws, ldo, opad, res, r_ws, ldr, rpad, strips, vec)
  if (nch == 1) {
    if (nco == 1) WINO_LAUNCH(1, 1); else if (nco == 2) WINO_LAUNCH(2, 1); else if (nco == 3) WINO_LAUNCH(3, 1);
    else WINO_LAUNCH(4, 1);
  } else if (nch == 2) {
    if (nco == 1) WINO_LAUNCH(1, 2); else if (nco == 2) WINO_LAUNCH(2, 2); else if (nco == 3) WINO_LAUNCH(3, 2);
    else WINO_LAUNCH(4, 2);
  } else {
    BNH_REQ(nch <= 2);  // C <= 64 in this kernel family
  }
#undef WINO_LAUNCH_A
#undef WINO_LAUNCH
  BNH_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"

// ================================================================== int8 Winograd F(2x2, 3x3) (WINO_S8)
// libbnneon's int8 Winograd (src/wino.c:26-227, the WINO_S8 op of src/rt_ops_dot.c:130-170), bit-identical:
//   V = B^T d B in fp32, quantised with ONE asymmetric scale per tile (over its 16 positions x C): s = range / 255,
//   zp = round(min / s) + 128, q = clamp(round(v / s) - zp) through the reference's magic-number FMA;
//   U = G g G^T quantised with ONE symmetric scale per output channel (over 16 x C) at load;
//   raw int32 position GEMMs on int8 MFMA, the integer output transform A^T M A, and per output
//   y = fma(zw[o], s zp, fma(float(Y) sw, s, b)), fp32 -> fp16, the fp16 LUT SiLU.
// Two kernels: k_wino8_in quantises the tiles (one wave per tile) into a scratch A8 [16][tiles][Cp] with the tile
// scales; k_wino8_out runs, per 16 tiles x 64 output channels, the 16 position GEMMs and the output transform in
// registers (a lane holds all 16 positions of 4 tiles for one channel).
struct bnh_w8w {
  int C, K, Cp, Kp;
  int8_t *U;         // [16][Kp][Cp], zero past C and K
  float *sw, *zw, *b;  // [Kp], [4][Kp], [Kp]
};

__global__ __launch_bounds__(256) void k_wino8_in(const float *__restrict__ x, long long x_ws, int H, int W, int C,
                                                  int Cp, int tw, int T, int Tp, int8_t *__restrict__ a8,
                                                  float *__restrict__ tsc, int B) {
  const int lane = threadIdx.x & 63;
  const long long gt = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);  // global tile index over all windows
  if (gt >= (long long)T * B) return;
  const int win = (int)(gt / T), t = (int)(gt % T), ti = t / tw, tj = t % tw;
  const float *xw = x + win * x_ws;
  auto tile_v = [&](int c, float v[16]) {
    float d[4][4], tm[4][4];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int cc = 0; cc < 4; cc++) {
        const int y = 2 * ti + r - 1, xx = 2 * tj + cc - 1;
        d[r][cc] = (y >= 0 && y < H && xx >= 0 && xx < W) ? xw[((long long)y * W + xx) * C + c] : 0.f;
      }
#pragma unroll
    for (int cc = 0; cc < 4; cc++) {
      tm[0][cc] = d[0][cc] - d[2][cc]; tm[1][cc] = d[1][cc] + d[2][cc];
      tm[2][cc] = d[2][cc] - d[1][cc]; tm[3][cc] = d[1][cc] - d[3][cc];
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      v[r * 4 + 0] = tm[r][0] - tm[r][2]; v[r * 4 + 1] = tm[r][1] + tm[r][2];
      v[r * 4 + 2] = tm[r][2] - tm[r][1]; v[r * 4 + 3] = tm[r][1] - tm[r][3];
    }
  };
  // pass 1: the tile's min / max over 16 positions x C, starting from 0 (FMIN / FMAX: any order gives the same)
  float mn = 0.f, mx = 0.f;
  for (int c = lane; c < C; c += 64) {
    float v[16];
    tile_v(c, v);
#pragma unroll
    for (int p = 0; p < 16; p++) { mn = bnh_fmin(mn, v[p]); mx = bnh_fmax(mx, v[p]); }
  }
  for (int off = 32; off; off >>= 1) {
    mn = bnh_fmin(mn, __shfl_xor(mn, off));
    mx = bnh_fmax(mx, __shfl_xor(mx, off));
  }
  float s = (mx - mn) > 0 ? (mx - mn) / 255.f : 1.f;
  if (s < 1e-30f) s = 1e-30f;
  const float inv = 1.f / s, zp = __builtin_rintf(mn * inv) + 128.f;
  const uint32_t zofs = 0x4B400000u + (uint32_t)bnh_cvtz_s32(zp);
  if (lane == 0) {
    tsc[2 * gt] = s;
    tsc[2 * gt + 1] = s * zp;
  }
  // pass 2: quantise; channels past C are zero
  int8_t *o = a8 + (long long)win * 16 * Tp * Cp + (long long)t * Cp;
  for (int c = lane; c < Cp; c += 64) {
    float v[16];
    if (c < C) tile_v(c, v);
#pragma unroll
    for (int p = 0; p < 16; p++) {
      int8_t q = 0;
      if (c < C) {
        const int32_t m = (int32_t)(__float_as_uint(__builtin_fmaf(v[p], inv, 12582912.0f)) - zofs);
        q = (int8_t)(m < -128 ? -128 : m > 127 ? 127 : m);
      }
      o[(long long)p * Tp * Cp + c] = q;
    }
  }
}

// 4 waves, each 16 output channels; 16 tiles per block (the MFMA rows)
__global__ __launch_bounds__(256) void k_wino8_out(const int8_t *__restrict__ a8, const float *__restrict__ tsc, int Cp,
                                                   int tw, int T, int Tp, const int8_t *__restrict__ U, int Kp, int K,
                                                   const float *__restrict__ sw, const float *__restrict__ zw,
                                                   const float *__restrict__ bias, int H, int W,
                                                   uint16_t *__restrict__ out, long long o_ws) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int win = blockIdx.z, t0 = blockIdx.x * 16, co = blockIdx.y * 64 + 16 * wave + (lane & 15);
  const int8_t *aw = a8 + (long long)win * 16 * Tp * Cp;
  const int ar = t0 + (lane & 15);  // this lane's A row (tile); rows past T hold zeros (Tp padding)
  v4i acc[16];
#pragma unroll
  for (int p = 0; p < 16; p++) {
    acc[p] = (v4i){0, 0, 0, 0};
    const int8_t *ap = aw + ((long long)p * Tp + ar) * Cp + 16 * (lane >> 4);
    const int8_t *bp = U + ((long long)p * Kp + (co < Kp ? co : Kp - 1)) * Cp + 16 * (lane >> 4);
    for (int k = 0; k < Cp; k += 64)
      acc[p] = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(const v4i *)(ap + k), *(const v4i *)(bp + k), acc[p], 0, 0, 0);
  }
  if (co >= K) return;
  const float swk = sw[co], bk = bias[co];
  const float zwk[4] = {zw[co], zw[Kp + co], zw[2 * Kp + co], zw[3 * Kp + co]};
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int t = t0 + 4 * (lane >> 4) + r;
    if (t >= T) continue;
    const float sa = tsc[2 * ((long long)win * T + t)], zs = tsc[2 * ((long long)win * T + t) + 1];
    uint32_t s0[4], s1[4];
#pragma unroll
    for (int cc = 0; cc < 4; cc++) {
      s0[cc] = ((uint32_t)acc[cc][r] + (uint32_t)acc[4 + cc][r]) + (uint32_t)acc[8 + cc][r];
      s1[cc] = ((uint32_t)acc[4 + cc][r] - (uint32_t)acc[8 + cc][r]) - (uint32_t)acc[12 + cc][r];
    }
    const uint32_t Y[4] = {(s0[0] + s0[1]) + s0[2], (s0[1] - s0[2]) - s0[3], (s1[0] + s1[1]) + s1[2],
                           (s1[1] - s1[2]) - s1[3]};
    const int ti = t / tw, tj = t % tw;
#pragma unroll
    for (int o = 0; o < 4; o++) {
      const int oy = 2 * ti + o / 2, ox = 2 * tj + o % 2;
      if (oy >= H || ox >= W) continue;
      const float inner = __builtin_fmaf((float)(int32_t)Y[o] * swk, sa, bk);
      const float y = __builtin_fmaf(zwk[o], zs, inner);
      out[win * o_ws + ((long long)oy * W + ox) * K + co] = hbits(silu_lut_h(f2h(y)));
    }
  }
}

extern "C" {

bnh_w8w *bnh_wino8_new(int C, int K, const float *w, const float *bias) {
  if (C <= 0 || K <= 0 || C % 8 || C > 2048 || K % 16 || K > 2048 || !w || !bias) {
    bnh_fail("bnh_wino8_new: C %d K %d: expected C %% 8 == 0, C <= 2048, K %% 16 == 0, K <= 2048 and both tensors",
             C, K);
    return nullptr;
  }
  const int Cp = (int)bnh_round_up(C, 64), Kp = K;
  float *U = (float *)malloc(sizeof(float) * 16 * (size_t)K * C);
  int8_t *hu = (int8_t *)calloc((size_t)16 * Kp * Cp, 1);
  float *hsw = (float *)calloc(Kp, 4), *hzw = (float *)calloc(4 * (size_t)Kp, 4);
  int32_t *wsum = (int32_t *)calloc(16 * (size_t)K, 4);
  bnh_w8w *P = (bnh_w8w *)calloc(1, sizeof *P);
  if (!U || !hu || !hsw || !hzw || !wsum || !P) {
    free(U); free(hu); free(hsw); free(hzw); free(wsum); free(P);
    bnh_fail("bnh_wino8_new: out of host memory");
    return nullptr;
  }
  // wino_pack (src/wino.c:26-88): the same fp32 operations in the same order
  for (int k = 0; k < K; k++)
    for (int c = 0; c < C; c++) {
      float g[3][3], tmp[4][3];
      for (int r = 0; r < 3; r++)
        for (int cc = 0; cc < 3; cc++) g[r][cc] = w[(((size_t)k * 3 + r) * 3 + cc) * C + c];
      for (int cc = 0; cc < 3; cc++) {
        tmp[0][cc] = g[0][cc];
        tmp[1][cc] = 0.5f * (g[0][cc] + g[1][cc] + g[2][cc]);
        tmp[2][cc] = 0.5f * (g[0][cc] - g[1][cc] + g[2][cc]);
        tmp[3][cc] = g[2][cc];
      }
      for (int r = 0; r < 4; r++) {
        const float u[4] = {tmp[r][0], 0.5f * (tmp[r][0] + tmp[r][1] + tmp[r][2]),
                            0.5f * (tmp[r][0] - tmp[r][1] + tmp[r][2]), tmp[r][2]};
        for (int cc = 0; cc < 4; cc++) U[((size_t)(r * 4 + cc) * K + k) * C + c] = u[cc];
      }
    }
  static const int AT[2][4] = {{1, 1, 1, 0}, {0, 1, -1, -1}};
  for (int k = 0; k < K; k++) {
    float mx = 0;
    for (int xi = 0; xi < 16; xi++)
      for (int c = 0; c < C; c++) mx = fmaxf(mx, fabsf(U[((size_t)xi * K + k) * C + c]));
    const float s = mx > 0 ? mx / 127.f : 1.f;
    hsw[k] = s;
    for (int xi = 0; xi < 16; xi++) {
      int32_t sum = 0;
      for (int c = 0; c < C; c++) {
        int v = (int)nearbyintf(U[((size_t)xi * K + k) * C + c] / s);
        v = v > 127 ? 127 : (v < -127 ? -127 : v);
        sum += v;
        hu[((size_t)xi * Kp + k) * Cp + c] = (int8_t)v;
      }
      wsum[xi * K + k] = sum;
    }
    for (int r = 0; r < 2; r++)
      for (int cc = 0; cc < 2; cc++) {
        long z = 0;
        for (int i = 0; i < 4; i++)
          for (int j = 0; j < 4; j++) z += (long)AT[r][i] * AT[cc][j] * wsum[(i * 4 + j) * K + k];
        hzw[(size_t)(r * 2 + cc) * Kp + k] = s * (float)z;
      }
  }
  free(U); free(wsum);
  P->C = C; P->K = K; P->Cp = Cp; P->Kp = Kp;
  bool ok = (P->U = (int8_t *)bnh_malloc((size_t)16 * Kp * Cp)) && (P->sw = (float *)bnh_malloc(4 * (size_t)Kp)) &&
            (P->zw = (float *)bnh_malloc(16 * (size_t)Kp)) && (P->b = (float *)bnh_malloc(4 * (size_t)Kp)) &&
            !bnh_memcpy_h2d(P->U, hu, (size_t)16 * Kp * Cp) && !bnh_memcpy_h2d(P->sw, hsw, 4 * (size_t)Kp) &&
            !bnh_memcpy_h2d(P->zw, hzw, 16 * (size_t)Kp) && !bnh_memcpy_h2d(P->b, bias, 4 * (size_t)K);
  free(hu); free(hsw); free(hzw);
  if (!ok) { bnh_wino8_free(P); return nullptr; }
  return P;
}

void bnh_wino8_free(bnh_w8w *P) {
  if (!P) return;
  if (P->U) (void)hipFree(P->U);
  if (P->sw) (void)hipFree(P->sw);
  if (P->zw) (void)hipFree(P->zw);
  if (P->b) (void)hipFree(P->b);
  free(P);
}

size_t bnh_wino8_work_bytes(int H, int W, int C, int B) {
  const long long T = (long long)((H + 1) / 2) * ((W + 1) / 2), Tp = bnh_round_up(T, 16);
  const long long Cp = bnh_round_up(C, 64);
  return (size_t)(B * (16 * Tp * Cp + 8 * T) + 256);
}

int bnh_wino_s8(const float *x, long long x_ws, int H, int W, const bnh_w8w *P, uint16_t *out, long long o_ws, int B,
                void *work, size_t work_bytes, void *stream) {
  BNH_REQ(x && P && out && work && H > 0 && W > 0 && B > 0);
  BNH_REQ(B == 1 || (x_ws >= (long long)H * W * P->C && o_ws >= (long long)H * W * P->K));
  BNH_REQ(work_bytes >= bnh_wino8_work_bytes(H, W, P->C, B));
  const int tw = (W + 1) / 2, T = ((H + 1) / 2) * tw, Tp = (int)bnh_round_up(T, 16);
  int8_t *a8 = (int8_t *)work;
  float *tsc = (float *)(a8 + (size_t)B * 16 * Tp * P->Cp);
  BNH_REQ(((uintptr_t)tsc & 3) == 0);
  hipStream_t st = bnh_stream(stream);
  // tile rows past T (up to Tp) of the scratch are read by the GEMM: zero them
  BNH_HIP(hipMemsetAsync(a8, 0, (size_t)B * 16 * Tp * P->Cp, st));
  hipLaunchKernelGGL(k_wino8_in, dim3((unsigned)bnh_ceil_div((long long)T * B, 4)), dim3(256), 0, st, x, x_ws, H, W,
                     P->C, P->Cp, tw, T, Tp, a8, tsc, B);
  BNH_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_wino8_out, dim3((unsigned)(Tp / 16), (unsigned)bnh_ceil_div(P->Kp, 64), (unsigned)B), dim3(256),
                     0, st, a8, tsc, P->Cp, tw, T, Tp, P->U, P->Kp, P->K, P->sw, P->zw, P->b, H, W, out, o_ws);
  BNH_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
