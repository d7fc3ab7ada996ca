// Depthwise convolutions of libbnneon on gfx950 (no MFMA: 2 k^2 flops per output against 2-4 bytes moved, so HBM
// bound): fp32 DWK (src/pc_kern_f32.c:163-334), fp32 DW3 (src/gemm_f32.c:213-441), fp16 DWK (src/pc_kern_f16.c:16-96)
// and fp16 DW3 (src/kern_f16.c:83-155), each bit-identical to the reference, plus this library's int8 depthwise
// (bnneon_hip.h states its specification). NHWC, channels across the lanes of a wavefront.
//
// Pass 1: a thread owns one channel of one "item" of an output row: a 4-pixel group (which the DWK forms compute
// with two chains, even and odd taps) or a tail pixel / pixel pair (one chain), so every output takes exactly the
// reference's chain for its position in the row. The thread loads its input window once into registers.
// Pass 2: the per-channel sums (the SE mean's input) are one serial fp32 chain per channel over the whole image in
// the reference's order; a thread per (window, channel) re-reads the outputs and adds them up that way.
#include <string.h>

#include "bnh_internal.h"
#include "bnh_num.h"

#include "bnh_f16.h"

// ------------------------------------------------------------------ the items of an output row
// DWK forms: items [0, g4/4) are 4-pixel groups, then (fp32) one item per tail pixel, or (fp16) a pixel pair when
// Wo % 4 >= 2 and a single pixel when Wo is odd. DW3 forms compute each pixel alike: items of up to 4 pixels.
struct Item { int px, n, split; };
BNH_DEV Item item_of(int it, int Wo, int form) {
  const int g4 = Wo & ~3, ng = g4 >> 2;
  Item r;
  if (form == 2) {  // DW3: groups of 4 (the last one shorter)
    r.px = it * 4;
    r.n = Wo - r.px < 4 ? Wo - r.px : 4;
    r.split = 0;
    return r;
  }
  if (it < ng) { r.px = it * 4; r.n = 4; r.split = 1; return r; }
  const int t = it - ng;
  if (form == 0) { r.px = g4 + t; r.n = 1; r.split = 0; return r; }  // fp32: single tail pixels
  const int two = (Wo - g4) & 2;                                        // fp16: a pair, then a single
  if (t == 0 && two) { r.px = g4; r.n = 2; r.split = 0; return r; }
  r.px = g4 + two;
  r.n = 1;
  r.split = 0;
  return r;
}
static int items_per_row(int Wo, int form) {
  const int g4 = Wo & ~3, ng = g4 >> 2, t = Wo - g4;
  if (form == 2) return (Wo + 3) / 4;
  if (form == 0) return ng + t;
  return ng + ((t & 2) ? 1 : 0) + (t & 1);
}

// ------------------------------------------------------------------ the grid
// A thread owns dw_ni(k) consecutive items of one output row and one channel (weights loaded once, input columns shared
// between neighbouring items reused from registers). Threads are numbered (window, row, strip, channel) across the
// whole grid, and blocks are taken in that order after the XCD remap, so one XCD walks consecutive rows of a window
// and finds the input rows they share in its L2.
// items per thread: 1 for 3 x 3 kernels (more threads in flight beat the reuse of weights), 4 for larger ones
__host__ __device__ constexpr int dw_ni(int k) { return k <= 3 ? 1 : 4; }
struct DwGrid { int ns, ni; double rC, rnc, rHo; };  // strips per row, items per strip; 1 / C, 1 / (ns C), 1 / Ho
struct DwPos { int c, it0, oy, win; bool ok; };
BNH_DEV DwPos dw_pos(int C, int Ho, long long total, DwGrid g) {
  const unsigned lb = bnh_xcd_block(blockIdx.x, gridDim.x);
  const long long i = (long long)lb * 256 + threadIdx.x;
  DwPos p;
  p.ok = i < total;
  const long long ii = p.ok ? i : 0;
  const int nc = g.ns * C;
  const int rowid = bnh_div(ii, nc, g.rnc), rem = (int)(ii - (long long)rowid * nc);
  const int strip = bnh_div(rem, C, g.rC);
  p.c = rem - strip * C;
  p.it0 = strip * g.ni;
  p.win = bnh_div(rowid, Ho, g.rHo);
  p.oy = rowid - p.win * Ho;
  return p;
}
static int dw_grid(int nitems, int ni, int C, int Ho, int B, unsigned *blocks, long long *total, DwGrid *g) {
  g->ni = ni;
  g->ns = (nitems + ni - 1) / ni;
  g->rC = 1.0 / C;
  g->rnc = 1.0 / ((double)g->ns * C);
  g->rHo = 1.0 / Ho;
  *total = (long long)B * Ho * g->ns * C;
  BNH_REQ(bnh_ceil_div(*total, 256) < (1LL << 31));
  *blocks = (unsigned)bnh_ceil_div(*total, 256);
  return 0;
}

// ------------------------------------------------------------------ fp32 DWK (form 0) and DW3 (form 2)
// The chains of one item's four outputs from its input window xv (rows ky, columns q S + kx for output q): DWK
// (src/pc_kern_f32.c:163-334) one chain per pixel, or for a 4-pixel group two per pixel (even and odd taps) added at
// the end; DW3 (src/gemm_f32.c:213-441) the three column partial sums. All four outputs are computed (those past the
// item's end from zeros, then dropped), so the chains have no branches between them.
// One input row ky of those chains (xr = row ky of the window): the chains run row by row, in the same order, whether
// the window sits in registers (k_dw_f32) or is read one row at a time (k_pwdw_f32). a / e / d: the chains' partial
// sums (DW3: the three column sums; DWK: even and odd taps, or one chain).
template <int K, int S, int FORM>
BNH_DEV void dw_row_f32(int ky, const float (&xr)[3 * S + K], const float (&wv)[K * K], float bias, bool split,
                        float (&a)[4], float (&e)[4], float (&d)[4]) {
#pragma unroll
  for (int q = 0; q < 4; q++) {
    if (FORM == 2) {
      const int o = q * S;
      if (ky == 0) {
        a[q] = __builtin_fmaf(wv[0], xr[o], bias);
        e[q] = wv[1] * xr[o + 1];
        d[q] = wv[2] * xr[o + 2];
      } else {
        a[q] = __builtin_fmaf(wv[3 * ky], xr[o], a[q]);
        e[q] = __builtin_fmaf(wv[3 * ky + 1], xr[o + 1], e[q]);
        d[q] = __builtin_fmaf(wv[3 * ky + 2], xr[o + 2], d[q]);
      }
    } else {
      if (ky == 0) {
        a[q] = bias;
        e[q] = 0.f;
      }
#pragma unroll
      for (int kx = 0; kx < K; kx++) {
        const int t = ky * K + kx;
        const float x = xr[q * S + kx];
        if (split && (t & 1)) e[q] = __builtin_fmaf(x, wv[t], e[q]);
        else a[q] = __builtin_fmaf(x, wv[t], a[q]);
      }
    }
  }
}
template <int K, int S, int FORM>
BNH_DEV void dw_finish_f32(bool split, const float (&a)[4], const float (&e)[4], const float (&d)[4], float (&v)[4]) {
#pragma unroll
  for (int q = 0; q < 4; q++) v[q] = FORM == 2 ? a[q] + (e[q] + d[q]) : split ? a[q] + e[q] : a[q];
}
template <int K, int S, int FORM>
BNH_DEV void dw_chains_f32(const float (&xv)[K][3 * S + K], const float (&wv)[K * K], float bias, bool split,
                           float (&v)[4]) {
  float a[4], e[4], d[4];
#pragma unroll
  for (int ky = 0; ky < K; ky++) dw_row_f32<K, S, FORM>(ky, xv[ky], wv, bias, split, a, e, d);
  dw_finish_f32<K, S, FORM>(split, a, e, d, v);
}

// DWK: input row oy*s - pt + h + ky, column px*s - pl + h + kx of the halo-h input. DW3: rows oy*s + ky, columns
// px*s + kx of the halo-1 input (pads 1), SiLU always.
template <int K, int S, int FORM>
__global__ __launch_bounds__(256) void k_dw_f32(const float *__restrict__ xp, long long x_ws, int Wp, int C, int pt,
                                                int pl, const float *__restrict__ w, const float *__restrict__ b,
                                                int act, float *__restrict__ out, long long o_ws, int Ho, int Wo,
                                                int nitems, long long total, DwGrid g) {
  __shared__ uint32_t tbl[256];
  bnh_silu_table(tbl);
  __syncthreads();
  const DwPos ps = dw_pos(C, Ho, total, g);
  if (!ps.ok) return;
  const int c = ps.c, oy = ps.oy, win = ps.win;
  constexpr int H = (K - 1) / 2, NC = 3 * S + K;  // input columns of a 4-pixel item
  const int iy0 = FORM == 2 ? oy * S : oy * S - pt + H;
  float wv[K * K];
#pragma unroll
  for (int t = 0; t < K * K; t++) wv[t] = w[(long long)t * C + c];
  const float bias = b[c];
  const float *xw = xp + win * x_ws + (long long)iy0 * Wp * C + c;
  float *ow = out + win * o_ws + (long long)oy * Wo * C + c;
  const long long rs = (long long)Wp * C;
#pragma unroll
  for (int j = 0; j < dw_ni(K); j++) {
    const int it = ps.it0 + j;
    if (it >= nitems) break;
    const Item item = item_of(it, Wo, FORM);
    const int ix0 = FORM == 2 ? item.px * S : item.px * S - pl + H;
    const float *x0 = xw + (long long)ix0 * C;
    // the item's whole input window first (columns past its last pixel's taps stay unread), so that its loads are
    // in flight together; a 4-pixel item (all but a row's last) reads all NC columns without a guard per load
    const int ncol = (item.n - 1) * S + K;
    float xv[K][NC];
    if (item.n == 4) {
#pragma unroll
      for (int ky = 0; ky < K; ky++)
#pragma unroll
        for (int kx = 0; kx < NC; kx++) xv[ky][kx] = x0[ky * rs + (long long)kx * C];
    } else {
#pragma unroll
      for (int ky = 0; ky < K; ky++)
#pragma unroll
        for (int kx = 0; kx < NC; kx++) xv[ky][kx] = kx < ncol ? x0[ky * rs + (long long)kx * C] : 0.f;
    }
    float v[4];
    dw_chains_f32<K, S, FORM>(xv, wv, bias, item.split, v);
    if (FORM == 2 || act == 1) {
#pragma unroll
      for (int q = 0; q < 4; q++) v[q] = bnh_silu_f32_t(v[q], tbl);
    }
    float *o = ow + (long long)item.px * C;
#pragma unroll
    for (int q = 0; q < 4; q++)
      if (q < item.n) o[(long long)q * C] = v[q];
  }
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// fp32 DW3 (halo-1 input, SiLU) on bands of R output rows: a thread owns a channel pair (8-byte loads) of a strip of
// 4 output pixels in a band of up to R rows. It loads each input row of the band's strip once and keeps the rows in
// registers while the band's output rows that share them are computed (k_dw_f32 loads the three input rows of every
// output row), and runs every output's chains through dw_row_f32, in its order. Loads are range-checked buffer loads
// on the haloed input: a strip past the row's end reads the next row (or, past the batch's last row, the buffer's
// out-of-range zeros) and stores nothing there; rows past a short last band are read and dropped.
template <int S, int R>
__global__ __launch_bounds__(256) void k_dw3_f32v(const float *__restrict__ xp, long long x_ws, unsigned x_len, int Wp,
                                                  int C, const float *__restrict__ w, const float *__restrict__ b,
                                                  float *__restrict__ out, long long o_ws, unsigned o_len, int Ho,
                                                  int Wo, long long total, DwGrid g) {
  __shared__ uint32_t tbl[256];
  bnh_silu_table(tbl);
  __syncthreads();
  const int nband = (Ho + R - 1) / R;
  const DwPos ps = dw_pos(C / 2, nband, total, g);
  if (!ps.ok) return;
  constexpr int NC = 3 * S + 3, NIN = (R - 1) * S + 3;  // input columns of the 4-pixel strip, input rows of a band
  const int c = 2 * ps.c, oy0 = ps.oy * R, px0 = ps.it0, nrows = Ho - oy0 < R ? Ho - oy0 : R;
  float wv[2][9], bias[2];
#pragma unroll
  for (int t = 0; t < 9; t++) {
    const float2 v = *(const float2 *)(w + (long long)t * C + c);
    wv[0][t] = v.x;
    wv[1][t] = v.y;
  }
  {
    const float2 v = *(const float2 *)(b + c);
    bias[0] = v.x;
    bias[1] = v.y;
  }
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void *)xp, 0, (int)x_len, 0x00020000);
  const __amdgpu_buffer_rsrc_t orr = __builtin_amdgcn_make_buffer_rsrc((void *)out, 0, (int)o_len, 0x00020000);
  // input row oy S + ky, column px S + kx of the halo-1 input (k_dw_f32's form 2)
  const int xo = 4 * ((int)(ps.win * x_ws) + (oy0 * S * Wp + px0 * S) * C + c);
  const int oo = 4 * ((int)(ps.win * o_ws) + (oy0 * Wo + px0) * C + c);
  const int rstep = 4 * Wp * C, cstep = 4 * C;
  float xin[NIN][NC][2];
#pragma unroll
  for (int i = 0; i < NIN; i++)
#pragma unroll
    for (int col = 0; col < NC; col++) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(xr, xo + i * rstep + col * cstep, 0, 0);
      xin[i][col][0] = bnh_float(v[0]);  // by value (a bit cast of an ext_vector element reads element 0)
      xin[i][col][1] = bnh_float(v[1]);
    }
#pragma unroll
  for (int r = 0; r < R; r++) {
    if (r >= nrows) break;
    float v[2][4];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      float pa[4], pe[4], pd[4];
#pragma unroll
      for (int ky = 0; ky < 3; ky++) {
        float row[NC];
#pragma unroll
        for (int col = 0; col < NC; col++) row[col] = xin[r * S + ky][col][j];
        dw_row_f32<3, S, 2>(ky, row, wv[j], bias[j], false, pa, pe, pd);
      }
      dw_finish_f32<3, S, 2>(false, pa, pe, pd, v[j]);
#pragma unroll
      for (int q = 0; q < 4; q++) v[j][q] = bnh_silu_f32_t(v[j][q], tbl);
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
      if (px0 + q >= Wo) break;
      const u32x2 st = {__builtin_bit_cast(uint32_t, v[0][q]), __builtin_bit_cast(uint32_t, v[1][q])};
      __builtin_amdgcn_raw_buffer_store_b64(st, orr, oo + r * 4 * Wo * C, q * cstep, 0);
    }
  }
}

// ------------------------------------------------------------------ PW_S8 expansion fused into the fp32 depthwise
// An int8 1x1 expansion (PW_S8: the int8 GEMM over rows that are already quantized, its fp32 dequant epilogue and
// activation, src/gemm_s8n.c:105-135) whose output only this depthwise conv reads. A block recomputes the expanded
// pixels one band of output rows needs into LDS (int8 MFMA), 16 channels at a time, and runs the depthwise chains of
// those channels from there, so the expanded tensor never reaches HBM. Every value is the one the two ops give: the
// int32 sums are exact in any order, the fp32 operations are the same ones in the same order as k_s8n_gemm's epilogue
// and k_dw_f32's chains, and cells outside the image hold the zero halo of the expansion's output buffer.
// Block = (window, band of TH output rows, one of gsplit parts of the 16-channel groups). It stages the band's int8
// rows, their scales and zero points and each pixel's LDS cell once, then walks its channel groups (each group's
// weights loaded one group ahead): expansion into LDS, barrier, depthwise, barrier. The expansion is VALU work
// (dequantisation and the exact SiLU of every expanded value); the kernel is bound by it, not by HBM.
// LDS (floats): the band's RIN = (TH - 1) S + K input rows x WL = (Wo - 1) S + K padded columns x 16 channels at a
// pixel stride of 20 (the four pixels 4 apart that one MFMA result store writes land in distinct banks) and a row
// stride RS with S RS = 16 (mod 64) (the four output rows one wavefront's depthwise reads cover land in distinct
// banks); 64 discard cells; then per band pixel (16 ntile of them) its scale, zero point and cell offset; then the
// int8 rows (Kp bytes each).
typedef int v4i __attribute__((ext_vector_type(4)));
template <int K, int S, int FORM, int KS>
__global__ __launch_bounds__(256) void k_pwdw_f32(const int8_t *__restrict__ q, long long q_ws,
                                                  const float *__restrict__ sa, long long sa_ws,
                                                  const int32_t *__restrict__ za, long long za_ws, int H, int W, int Kp,
                                                  const int8_t *__restrict__ wt, const float *__restrict__ sw,
                                                  const int32_t *__restrict__ cs, const float *__restrict__ pb, int pact,
                                                  int C, int pt, int pl, const float *__restrict__ w,
                                                  const float *__restrict__ b, int dact, float *__restrict__ out,
                                                  long long o_ws, int Ho, int Wo, int nit, int TH, int nband,
                                                  int gsplit, int WL, int RS, int sz_off, int npx, double rW) {
  constexpr int CG = 16, PS = 20;  // channels per group, pixel stride
  extern __shared__ float xs[];
  __shared__ uint32_t tbl[256];
  bnh_silu_table(tbl);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const unsigned lb = bnh_xcd_block(blockIdx.x, gridDim.x);
  const int part = (int)(lb % gsplit);
  const unsigned rest = lb / gsplit;
  const int band = (int)(rest % nband), win = (int)(rest / nband);
  const int ncg = C / CG, g0 = part * ncg / gsplit, g1 = (part + 1) * ncg / gsplit;
  const int oy0 = band * TH, THb = Ho - oy0 < TH ? Ho - oy0 : TH;
  const int RIN = (THb - 1) * S + K, ybase = oy0 * S - pt;  // LDS row r holds image row ybase + r
  const int y0 = ybase > 0 ? ybase : 0, y1 = ybase + RIN < H ? ybase + RIN : H;
  const int xr = pl + W < WL ? pl + W : WL;  // LDS columns [pl, xr) hold image columns [0, xr - pl)
  const int p0 = y0 * W, np = (y1 - y0) * W, ntile = (np + 15) / 16;
  float *s_sa = xs + sz_off;  // [npx] (npx >= 16 ntile of every band)
  uint32_t *s_z = (uint32_t *)(s_sa + npx);
  int *s_off = (int *)(s_z + npx);
  int8_t *s_q = (int8_t *)(s_off + npx);  // [np][Kp]
  const int trash = sz_off - 64;          // discard cells
  // stage: the band's int8 rows (16-byte chunks), each pixel's scale, zero point and LDS cell (discard cells for the
  // pixels of the last tile past the band)
  {
    const int8_t *qw = q + win * q_ws + (long long)p0 * Kp;
    const int nch = np * Kp / 16;
    for (int i = threadIdx.x; i < nch; i += 256) *(v4i *)(s_q + 16 * i) = *(const v4i *)(qw + 16 * i);
    for (int i = threadIdx.x; i < 16 * ntile; i += 256) {
      const int p = p0 + (i < np ? i : np - 1);
      s_sa[i] = sa[win * sa_ws + p];
      s_z[i] = (uint32_t)za[win * za_ws + p];
      const int y = bnh_div(p, W, rW), x = p - y * W;
      s_off[i] = i < np && pl + x < WL ? (y - ybase) * RS + (pl + x) * PS : trash;
    }
  }
  // zeros of the cells outside the image (rows above and below it, then the columns left and right of it): written
  // once, no channel group's expansion touches them
  {
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    const int top = (y0 - ybase) * RS, bot = (y1 - ybase) * RS, end = RIN * RS;
    for (int i = 4 * threadIdx.x; i < top; i += 1024) *(float4 *)(xs + i) = z4;
    for (int i = bot + 4 * threadIdx.x; i < end; i += 1024) *(float4 *)(xs + i) = z4;
    const int nh = WL - (xr - pl);  // halo columns per row
    const int n = (y1 - y0) * nh * (CG / 4);
    for (int i = threadIdx.x; i < n; i += 256) {
      const int c4 = i % (CG / 4), cell = i / (CG / 4);
      const int r = cell / nh, j = cell - r * nh;
      const int xl = j < pl ? j : xr + (j - pl);
      *(float4 *)(xs + (y0 - ybase + r) * RS + xl * PS + 4 * c4) = z4;
    }
  }
  constexpr int NC = 3 * S + K;
  const int c = threadIdx.x % CG, nl = lane & 15, kc = (lane >> 4) * 16;
  const int npos = THb * nit;
  // pos / THb as (pos + 0.5) / THb in float: its distance to the nearest integer, >= 0.5 / THb, exceeds the product's
  // error, < npos 2^-23 / THb, for npos < 2^22 (the plan keeps npos < 2^16)
  const float rth = 1.f / (float)THb;
  float *ow = out + win * o_ws + (long long)oy0 * Wo * C + c;
  // the first group's expansion constants and weight fragments (later groups': loaded one group ahead)
  float swn = sw[16 * g0 + nl], bn = pb[16 * g0 + nl];
  int32_t csn = cs[16 * g0 + nl];
  v4i bf[KS];
#pragma unroll
  for (int k = 0; k < KS; k++)
    bf[k] = 64 * k + kc < Kp ? *(const v4i *)(wt + (long long)(16 * g0 + nl) * Kp + 64 * k + kc) : (v4i){0, 0, 0, 0};
  __syncthreads();  // the SiLU table, the staged rows, the zeros
  for (int g = g0; g < g1; g++) {
    const int c0 = 16 * g;
    // this group's depthwise weights: consumed after the expansion, which hides their latency
    float wv[K * K];
#pragma unroll
    for (int t = 0; t < K * K; t++) wv[t] = w[(long long)t * C + c0 + c];
    const float bias = b[c0 + c];
    // expansion of the band's pixels, channels c0 .. c0 + 15: lane l holds pixels 16 t + 4 (l >> 4) .. + 3 of channel
    // c0 + (l & 15)
    for (int t = wave; t < ntile; t += 4) {
      const int8_t *arow = s_q + (16 * t + nl) * Kp + kc;
      v4i acc = {0, 0, 0, 0};
#pragma unroll
      for (int k = 0; k < KS; k++)
        if (64 * k < Kp) {
          const v4i a = 64 * k + kc < Kp && 16 * t + nl < np ? *(const v4i *)(arow + 64 * k) : (v4i){0, 0, 0, 0};
          acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bf[k], acc, 0, 0, 0);
        }
      const int pr0 = 16 * t + 4 * (lane >> 4);
      const float4 s4 = *(const float4 *)(s_sa + pr0);
      const uint4 z4 = *(const uint4 *)(s_z + pr0);
      const int4 o4 = *(const int4 *)(s_off + pr0);
      const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
      const uint32_t zv[4] = {z4.x, z4.y, z4.z, z4.w};
      const int ov[4] = {o4.x, o4.y, o4.z, o4.w};
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int32_t cq = (int32_t)((uint32_t)acc[r] - (uint32_t)csn * zv[r]);
        const float f = (float)cq;
        const float scl = swn * sv[r];
        const float yv = f * scl;
        v[r] = yv + bn;
      }
      if (pact == 1) {
#pragma unroll
        for (int r = 0; r < 4; r++) v[r] = bnh_silu_f32_t(v[r], tbl);
      } else if (pact == 2) {
#pragma unroll
        for (int r = 0; r < 4; r++) v[r] = bnh_relu_f32(v[r]);
      }
#pragma unroll
      for (int r = 0; r < 4; r++) xs[ov[r] + nl] = v[r];
    }
    __syncthreads();
    // the next group's expansion constants, in flight during this group's depthwise
    if (g + 1 < g1) {
      const int n = 16 * (g + 1) + nl;
      swn = sw[n];
      bn = pb[n];
      csn = cs[n];
#pragma unroll
      for (int k = 0; k < KS; k++)
        bf[k] = 64 * k + kc < Kp ? *(const v4i *)(wt + (long long)n * Kp + 64 * k + kc) : (v4i){0, 0, 0, 0};
    }
    // the depthwise chains: thread = (channel c, position), positions = (item, output row) with the row fastest
    for (int pos = threadIdx.x / CG; pos < npos; pos += 256 / CG) {
      const int it = (int)(((float)pos + 0.5f) * rth), row = pos - it * THb;
      const Item item = item_of(it, Wo, FORM);
      const float *x0 = xs + row * S * RS + item.px * S * PS + c;
      float pa[4], pe[4], pd[4], v[4];
#pragma unroll
      for (int ky = 0; ky < K; ky++) {  // one input row at a time
        // all NC columns, unguarded: those past the item's (item.n - 1) S + K feed only its outputs q >= item.n, which
        // are dropped, and read at most 3 S cells past the row's WL, within the allocation (the next row, or the
        // discard cells and per-pixel arrays after the last row: 60 S - 5 floats past RIN RS at most, < 64 + 12 + 16)
        float xr_[NC];
#pragma unroll
        for (int kx = 0; kx < NC; kx++) xr_[kx] = x0[ky * RS + kx * PS];
        dw_row_f32<K, S, FORM>(ky, xr_, wv, bias, item.split, pa, pe, pd);
      }
      dw_finish_f32<K, S, FORM>(item.split, pa, pe, pd, v);
      if (FORM == 2 || dact == 1) {
#pragma unroll
        for (int qq = 0; qq < 4; qq++) v[qq] = bnh_silu_f32_t(v[qq], tbl);
      }
      float *o = ow + ((long long)row * Wo + item.px) * C + c0;
#pragma unroll
      for (int qq = 0; qq < 4; qq++)
        if (qq < item.n) o[(long long)qq * C] = v[qq];
    }
    __syncthreads();  // the next group's expansion overwrites the cells
  }
}

// ------------------------------------------------------------------ fp16 DWK (form 1) and DW3 (form 2)
template <int K, int S, int FORM>
__global__ __launch_bounds__(256) void k_dw_f16(const h16 *__restrict__ xp, long long x_ws, int Wp, int C, int pt,
                                                int pl, const h16 *__restrict__ w, const h16 *__restrict__ b, int act,
                                                h16 *__restrict__ out, long long o_ws, int Ho, int Wo, int nitems,
                                                long long total, DwGrid g) {
  const DwPos ps = dw_pos(C, Ho, total, g);
  if (!ps.ok) return;
  const int c = ps.c, oy = ps.oy, win = ps.win;
  constexpr int H = (K - 1) / 2;
  const int iy0 = FORM == 2 ? oy * S - pt + 1 : oy * S - pt + H;
  h16 wv[K * K];
#pragma unroll
  for (int t = 0; t < K * K; t++) wv[t] = w[(long long)t * C + c];
  const h16 bias = b[c];
  const h16 *xw = xp + win * x_ws + (long long)iy0 * Wp * C + c;
  h16 *ow = out + win * o_ws + (long long)oy * Wo * C + c;
#pragma unroll
  for (int j = 0; j < dw_ni(K); j++) {
    const int it = ps.it0 + j;
    if (it >= nitems) break;
    const Item item = item_of(it, Wo, FORM);
    const int ix0 = FORM == 2 ? item.px * S - pl + 1 : item.px * S - pl + H;
    const h16 *x0 = xw + (long long)ix0 * C;
    h16 v[4];
#pragma unroll
    for (int q = 0; q < 4; q++) v[q] = (h16)0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      if (q >= item.n) break;
      if (FORM == 2) {
        const h16 *r0 = x0 + (long long)q * S * C, *r1 = r0 + (long long)Wp * C, *r2 = r1 + (long long)Wp * C;
        h16 a = hfma(r0[0], wv[0], bias);
        h16 a2 = r0[C] * wv[1];
        a = hfma(r0[2 * C], wv[2], a);
        a2 = hfma(r1[0], wv[3], a2);
        a = hfma(r1[C], wv[4], a);
        a2 = hfma(r1[2 * C], wv[5], a2);
        a = hfma(r2[0], wv[6], a);
        a2 = hfma(r2[C], wv[7], a2);
        a = hfma(r2[2 * C], wv[8], a);
        v[q] = silu_lut_h(a + a2);
      } else {
        h16 a = bias, e = (h16)0.0f;
#pragma unroll
        for (int ky = 0; ky < K; ky++)
#pragma unroll
          for (int kx = 0; kx < K; kx++) {
            const int t = ky * K + kx;
            const h16 xv = x0[((long long)ky * Wp + q * S + kx) * C];
            if (item.split && (t & 1)) e = hfma(xv, wv[t], e);
            else a = hfma(xv, wv[t], a);
          }
        h16 y = item.split ? a + e : a;
        if (act == 1) y = silu_lut_h(y);
        v[q] = y;
      }
    }
    h16 *o = ow + (long long)item.px * C;
#pragma unroll
    for (int q = 0; q < 4; q++)
      if (q < item.n) o[(long long)q * C] = v[q];
  }
}

// The same on channel pairs (C even): a thread owns two adjacent channels and runs their two chains in the lanes of
// packed fp16 instructions (each lane one IEEE fp16 operation, the same roundings as k_dw_f16), 4-byte loads and
// stores, the LUT SiLU on both halves with its table in LDS.
template <int K, int S, int FORM>
__global__ __launch_bounds__(256) void k_dw_f16p(const h16 *__restrict__ xp, long long x_ws, int Wp, int C, int pt,
                                                 int pl, const h16 *__restrict__ w, const h16 *__restrict__ b, int act,
                                                 h16 *__restrict__ out, long long o_ws, int Ho, int Wo, int nitems,
                                                 long long total, DwGrid g) {
  __shared__ uint32_t s_t01[16];
  __shared__ uint16_t s_t2[16];
  if (threadIdx.x < 16) {
    s_t01[threadIdx.x] = (uint32_t)k_silu_c0[threadIdx.x] | ((uint32_t)k_silu_c1[threadIdx.x] << 16);
    s_t2[threadIdx.x] = k_silu_c2[threadIdx.x];
  }
  __syncthreads();
  const DwPos ps = dw_pos(C / 2, Ho, total, g);
  if (!ps.ok) return;
  const int c = 2 * ps.c, oy = ps.oy, win = ps.win;
  constexpr int H = (K - 1) / 2;
  const int iy0 = FORM == 2 ? oy * S - pt + 1 : oy * S - pt + H;
  auto ld2 = [](const h16 *p) { return __builtin_bit_cast(h2, *(const uint32_t *)p); };
  h2 wv[K * K];
#pragma unroll
  for (int t = 0; t < K * K; t++) wv[t] = ld2(w + (long long)t * C + c);
  const h2 bias = ld2(b + c);
  const h16 *xw = xp + win * x_ws + (long long)iy0 * Wp * C + c;
  h16 *ow = out + win * o_ws + (long long)oy * Wo * C + c;
#pragma unroll
  for (int j = 0; j < dw_ni(K); j++) {
    const int it = ps.it0 + j;
    if (it >= nitems) break;
    const Item item = item_of(it, Wo, FORM);
    const int ix0 = FORM == 2 ? item.px * S - pl + 1 : item.px * S - pl + H;
    const h16 *x0 = xw + (long long)ix0 * C;
    h2 v[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      if (q >= item.n) break;
      if (FORM == 2) {
        const h16 *r0 = x0 + (long long)q * S * C, *r1 = r0 + (long long)Wp * C, *r2 = r1 + (long long)Wp * C;
        h2 a = __builtin_elementwise_fma(ld2(r0), wv[0], bias);
        h2 a2 = ld2(r0 + C) * wv[1];
        a = __builtin_elementwise_fma(ld2(r0 + 2 * C), wv[2], a);
        a2 = __builtin_elementwise_fma(ld2(r1), wv[3], a2);
        a = __builtin_elementwise_fma(ld2(r1 + C), wv[4], a);
        a2 = __builtin_elementwise_fma(ld2(r1 + 2 * C), wv[5], a2);
        a = __builtin_elementwise_fma(ld2(r2), wv[6], a);
        a2 = __builtin_elementwise_fma(ld2(r2 + C), wv[7], a2);
        a = __builtin_elementwise_fma(ld2(r2 + 2 * C), wv[8], a);
        v[q] = silu2_lut(a + a2, s_t01, s_t2);
      } else {
        h2 a = bias, e = (h2){(h16)0.0f, (h16)0.0f};
#pragma unroll
        for (int ky = 0; ky < K; ky++)
#pragma unroll
          for (int kx = 0; kx < K; kx++) {
            const int t = ky * K + kx;
            const h2 xv = ld2(x0 + ((long long)ky * Wp + q * S + kx) * C);
            if (item.split && (t & 1)) e = __builtin_elementwise_fma(xv, wv[t], e);
            else a = __builtin_elementwise_fma(xv, wv[t], a);
          }
        h2 y = item.split ? a + e : a;
        if (act == 1) y = silu2_lut(y, s_t01, s_t2);
        v[q] = y;
      }
    }
    h16 *o = ow + (long long)item.px * C;
#pragma unroll
    for (int q = 0; q < 4; q++)
      if (q < item.n) *(uint32_t *)(o + (long long)q * C) = __builtin_bit_cast(uint32_t, v[q]);
  }
}

// The same on channel quads (C % 4 == 0, 8-byte aligned data): a thread owns CP packed pairs (the fp16 DWK launch
// takes one, the fp16 DW3 launch two) of a strip of NP output pixels (whole items) in a band of up to R output rows.
// It loads each input row of the band's strip once (4- or 8-byte buffer loads: the lane's row in the vector offset,
// the column step in the scalar one; the input is
// haloed, so no checks: a strip past the row's end reads the next row or, at the batch's end, the buffer's
// out-of-range zeros, and stores nothing there) and keeps the rows in registers while the band's output rows that
// share them are computed. Each pixel runs its chains row by row in the reference's tap order: the two chains of a
// 4-pixel group (even / odd taps; DW3: its a / a2 chains, a2 opened by a product) or the one chain of a DWK tail
// pixel. ALL: every pixel of the strip lies in a 4-pixel group.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// a packed pair from a 32-bit word (by value: clang's __builtin_bit_cast of an ext_vector element reads element 0)
BNH_DEV h2 h2_bits(uint32_t u) { return __builtin_bit_cast(h2, u); }
// output rows per band: input rows shared by more outputs against registers and the number of waves
__host__ __device__ constexpr int dw_f16v_np(int k, int s) { return k == 3 && s == 1 ? 8 : 4; }
// (5 x 5 stride 1: 6 rows, 3.3 input loads per output pair where 4-row bands take 4; the 24 x 64 C = 672 launch of 64
// windows 0.0914 -> 0.0856 ms; 8 rows the same, 10 and more spill)
// the DW3 form on channel quads (two pairs a thread): 4-pixel strips at either stride (3x3 s1 with 8-pixel strips held
// 141 VGPRs and 3 waves per SIMD, with 4 it holds 95 and 5: the v2.4-shaped net 3.815 -> 3.764 ms on one stream)
__host__ __device__ constexpr int dw3_f16v_np(int s) { return 4; }
__host__ __device__ constexpr int dw_f16v_rows(int k, int s) { return k == 5 && s == 1 ? 6 : s == 1 ? 4 : 2; }

template <int K, int S, int FORM, int NP, int R, int CP, bool ALL>
BNH_DEV void dw_f16v_band(__amdgpu_buffer_rsrc_t xr, int xo, int rstep, int cstep, int px0, int g4, int nrows,
                          const h2 (&wv)[K * K][CP], const h2 (&bias)[CP], bool silu, const uint32_t *t01,
                          const uint16_t *t2, __amdgpu_buffer_rsrc_t orr, int oo, int ostep, int Wo) {
  constexpr int NCOL = (NP - 1) * S + K, NIN = (R - 1) * S + K;
  // every row of a full band: the rows a short last band does not use are read (from the next window, or as the
  // buffer's out-of-range zeros) and dropped
  h2 xin[NIN][NCOL][CP];
#pragma unroll
  for (int i = 0; i < NIN; i++)
#pragma unroll
    for (int col = 0; col < NCOL; col++) {
      // a strip past the row's end (not ALL) keeps its whole offset in the vector operand, the range-checked one
      if (CP == 2) {
        const u32x2 v = ALL ? __builtin_amdgcn_raw_buffer_load_b64(xr, xo + i * rstep, col * cstep, 0)
                            : __builtin_amdgcn_raw_buffer_load_b64(xr, xo + i * rstep + col * cstep, 0, 0);
        xin[i][col][0] = h2_bits(v[0]);
        xin[i][col][CP - 1] = h2_bits(v[1]);
      } else {
        const uint32_t v = ALL ? __builtin_amdgcn_raw_buffer_load_b32(xr, xo + i * rstep, col * cstep, 0)
                               : __builtin_amdgcn_raw_buffer_load_b32(xr, xo + i * rstep + col * cstep, 0, 0);
        xin[i][col][0] = h2_bits(v);
      }
    }
  const h2 z = (h2){(h16)0.0f, (h16)0.0f};
#pragma unroll
  for (int r = 0; r < R; r++) {
    if (r >= nrows) break;
    h2 a[NP][CP], e[NP][CP];
#pragma unroll
    for (int q = 0; q < NP; q++) {
      const bool split = FORM == 2 || ALL || px0 + q < g4;
#pragma unroll
      for (int j = 0; j < CP; j++) {
        a[q][j] = bias[j];
        e[q][j] = z;
      }
#pragma unroll
      for (int ky = 0; ky < K; ky++)
#pragma unroll
        for (int kx = 0; kx < K; kx++) {
          const int t = ky * K + kx;
#pragma unroll
          for (int j = 0; j < CP; j++) {
            const h2 x = xin[r * S + ky][q * S + kx][j];
            if (FORM == 2 && t == 1) e[q][j] = x * wv[t][j];
            else if (split && (t & 1)) e[q][j] = __builtin_elementwise_fma(x, wv[t][j], e[q][j]);
            else a[q][j] = __builtin_elementwise_fma(x, wv[t][j], a[q][j]);
          }
        }
#pragma unroll
      for (int j = 0; j < CP; j++) {
        h2 y = split ? a[q][j] + e[q][j] : a[q][j];
        if (silu) y = silu2_lut(y, t01, t2);
        a[q][j] = y;
      }
    }
#pragma unroll
    for (int q = 0; q < NP; q++) {
      if (px0 + q >= Wo) break;
      if (CP == 2) {
        const u32x2 v = {__builtin_bit_cast(uint32_t, a[q][0]), __builtin_bit_cast(uint32_t, a[q][CP - 1])};
        __builtin_amdgcn_raw_buffer_store_b64(v, orr, oo + r * ostep, q * cstep, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, a[q][0]), orr, oo + r * ostep, q * cstep, 0);
      }
    }
  }
}

template <int K, int S, int FORM, int NP, int R, int CP>
__global__ __launch_bounds__(256) void k_dw_f16v(const h16 *__restrict__ xp, long long x_ws, unsigned x_len, int Wp,
                                                 int C, int pt, int pl, const h16 *__restrict__ w,
                                                 const h16 *__restrict__ b, int act, h16 *__restrict__ out,
                                                 long long o_ws, unsigned o_len, int Ho, int Wo, long long total,
                                                 DwGrid g) {
  __shared__ uint32_t s_t01[16];
  __shared__ uint16_t s_t2[16];
  if (threadIdx.x < 16) {
    s_t01[threadIdx.x] = (uint32_t)k_silu_c0[threadIdx.x] | ((uint32_t)k_silu_c1[threadIdx.x] << 16);
    s_t2[threadIdx.x] = k_silu_c2[threadIdx.x];
  }
  __syncthreads();
  const int nband = (Ho + R - 1) / R;
  const DwPos ps = dw_pos(C / (2 * CP), nband, total, g);
  if (!ps.ok) return;
  const int c = 2 * CP * ps.c, oy0 = ps.oy * R, px0 = ps.it0, nrows = Ho - oy0 < R ? Ho - oy0 : R;
  constexpr int HH = (K - 1) / 2;
  const int iy0 = FORM == 2 ? oy0 * S - pt + 1 : oy0 * S - pt + HH;
  const int ix0 = FORM == 2 ? px0 * S - pl + 1 : px0 * S - pl + HH;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void *)w, 0, K * K * C * 2, 0x00020000);
  h2 wv[K * K][CP], bias[CP];
#pragma unroll
  for (int t = 0; t < K * K; t++) {
    if (CP == 2) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(wr, 2 * c, t * C * 2, 0);
      wv[t][0] = h2_bits(v[0]);
      wv[t][CP - 1] = h2_bits(v[1]);
    } else {
      wv[t][0] = h2_bits(__builtin_amdgcn_raw_buffer_load_b32(wr, 2 * c, t * C * 2, 0));
    }
  }
  if (CP == 2) {
    const uint2 v = *(const uint2 *)(b + c);
    bias[0] = __builtin_bit_cast(h2, v.x);
    bias[CP - 1] = __builtin_bit_cast(h2, v.y);
  } else {
    bias[0] = __builtin_bit_cast(h2, *(const uint32_t *)(b + c));
  }
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void *)xp, 0, (int)x_len, 0x00020000);
  const __amdgpu_buffer_rsrc_t orr = __builtin_amdgcn_make_buffer_rsrc((void *)out, 0, (int)o_len, 0x00020000);
  const int xo = 2 * ((int)(ps.win * x_ws) + (iy0 * Wp + ix0) * C + c);
  const int oo = 2 * ((int)(ps.win * o_ws) + (oy0 * Wo + px0) * C + c);
  const int g4 = FORM == 2 ? Wo : Wo & ~3;
  const bool silu = FORM == 2 || act == 1;
  if (px0 + NP <= g4)
    dw_f16v_band<K, S, FORM, NP, R, CP, true>(xr, xo, 2 * Wp * C, 2 * C, px0, g4, nrows, wv, bias, silu, s_t01, s_t2, orr,
                                          oo, 2 * Wo * C, Wo);
  else
    dw_f16v_band<K, S, FORM, NP, R, CP, false>(xr, xo, 2 * Wp * C, 2 * C, px0, g4, nrows, wv, bias, silu, s_t01, s_t2, orr,
                                           oo, 2 * Wo * C, Wo);
}

// ------------------------------------------------------------------ channel sums (pass 2)
// The reference adds the outputs of each channel into one fp32 sum, row after row, in terms that depend on the kernel:
//   form 0 (fp32 DWK): per row the 4-pixel groups (o0 + o1) + (o2 + o3), then each tail pixel;
//   form 2 (fp32 DW3): every pixel in raster order;
//   form 1 (fp16 DWK): per row fp16 group sums (o0 + o1) + (o2 + o3), then an fp16 pair, then a single, widened;
//   form 3 (fp16 DW3): per row an fp16 running sum over the row, widened at the row's end.
// The sum is one dependent chain per channel. A block owns one window and a slab of <= 64 channels: all its waves
// compute the terms of a chunk of rows into LDS (4 channels per item, vector loads), then wave 0 (one lane per
// channel) adds them in order while the other waves compute the next chunk into the second buffer.
template <int FORM>
__device__ __forceinline__ int cs_terms(int Wo) {
  if (FORM == 0) return Wo / 4 + Wo % 4;
  if (FORM == 2) return Wo;
  if (FORM == 1) return Wo / 4 + ((Wo % 4) >> 1) + (Wo & 1);
  return 1;
}

struct f4 { float v[4]; };

BNH_DEV f4 cs_ld(const float *p) {
  const float4 t = *(const float4 *)p;
  return f4{{t.x, t.y, t.z, t.w}};
}
BNH_DEV void cs_ld(const h16 *p, h16 (&o)[4]) {
  const uint2 t = *(const uint2 *)p;
  o[0] = hfrom((uint16_t)(t.x & 0xffffu)); o[1] = hfrom((uint16_t)(t.x >> 16));
  o[2] = hfrom((uint16_t)(t.y & 0xffffu)); o[3] = hfrom((uint16_t)(t.y >> 16));
}

// term j of a row (row points at the row's first pixel, channel c0 of the 4) for 4 channels
template <int FORM>
BNH_DEV f4 cs_term(const float *row, int C, int Wo, int j) {
  const int g4 = Wo / 4;
  if (FORM == 0 && j < g4) {
    const f4 a = cs_ld(row + (long long)(4 * j) * C), b = cs_ld(row + (long long)(4 * j + 1) * C);
    const f4 c = cs_ld(row + (long long)(4 * j + 2) * C), d = cs_ld(row + (long long)(4 * j + 3) * C);
    f4 r;
#pragma unroll
    for (int q = 0; q < 4; q++) r.v[q] = (a.v[q] + b.v[q]) + (c.v[q] + d.v[q]);
    return r;
  }
  const int ox = FORM == 0 ? 4 * g4 + (j - g4) : j;
  return cs_ld(row + (long long)ox * C);
}
template <int FORM>
BNH_DEV f4 cs_term(const h16 *row, int C, int Wo, int j) {
  f4 r;
  h16 a[4], b[4], c[4], d[4];
  if (FORM == 3) {
    h16 rs[4] = {(h16)0.0f, (h16)0.0f, (h16)0.0f, (h16)0.0f};
    for (int ox = 0; ox < Wo; ox++) {
      cs_ld(row + (long long)ox * C, a);
#pragma unroll
      for (int q = 0; q < 4; q++) rs[q] = rs[q] + a[q];
    }
#pragma unroll
    for (int q = 0; q < 4; q++) r.v[q] = (float)rs[q];
    return r;
  }
  const int g4 = Wo / 4, np = (Wo % 4) >> 1;
  if (j < g4) {
    cs_ld(row + (long long)(4 * j) * C, a);
    cs_ld(row + (long long)(4 * j + 1) * C, b);
    cs_ld(row + (long long)(4 * j + 2) * C, c);
    cs_ld(row + (long long)(4 * j + 3) * C, d);
#pragma unroll
    for (int q = 0; q < 4; q++) r.v[q] = (float)((a[q] + b[q]) + (c[q] + d[q]));
  } else if (j < g4 + np) {
    cs_ld(row + (long long)(4 * g4) * C, a);
    cs_ld(row + (long long)(4 * g4 + 1) * C, b);
#pragma unroll
    for (int q = 0; q < 4; q++) r.v[q] = (float)(a[q] + b[q]);
  } else {
    cs_ld(row + (long long)(Wo - 1) * C, a);
#pragma unroll
    for (int q = 0; q < 4; q++) r.v[q] = (float)a[q];
  }
  return r;
}

template <typename T, int FORM>
__global__ __launch_bounds__(256) void k_chsum(const T *__restrict__ out, long long o_ws, int C, int Ho, int Wo, int R,
                                               float *__restrict__ chsum, long long cs_ws) {
  extern __shared__ float tb[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c0 = blockIdx.x * 64, S = C - c0 < 64 ? C - c0 : 64, S4 = S / 4, win = blockIdx.y;
  const int Tn = cs_terms<FORM>(Wo), per = R * Tn * S, nch = (Ho + R - 1) / R;
  const T *o = out + win * o_ws + c0;
  // a chunk's terms: each thread takes items t0, t0 + nt, ...; CB items' loads are issued before any of their LDS
  // stores, so that a thread keeps CB loads (4 CB for the 4-pixel terms) in flight
  constexpr int CB = FORM == 2 ? 16 : 4;
  auto load = [&](int ch, int t0, int nt) {
    const int rows = Ho - ch * R < R ? Ho - ch * R : R;
    float *buf = tb + (ch & 1) * per;
    const int n = rows * Tn * S4;
    for (int base = t0; base < n; base += CB * nt) {
      f4 v[CB];
#pragma unroll
      for (int u = 0; u < CB; u++) {
        const int it = base + u * nt;
        if (it < n) {
          const int c4 = it % S4, j = (it / S4) % Tn, r = it / (S4 * Tn);
          v[u] = cs_term<FORM>(o + (long long)(ch * R + r) * Wo * C + 4 * c4, C, Wo, j);
        }
      }
#pragma unroll
      for (int u = 0; u < CB; u++) {
        const int it = base + u * nt;
        if (it < n) {
          const int c4 = it % S4, j = (it / S4) % Tn, r = it / (S4 * Tn);
          *(float4 *)(buf + (r * Tn + j) * S + 4 * c4) = make_float4(v[u].v[0], v[u].v[1], v[u].v[2], v[u].v[3]);
        }
      }
    }
  };
  load(0, tid, 256);
  __syncthreads();
  float cs = 0.f;
  for (int ch = 0; ch < nch; ch++) {
    if (wave != 0) {
      if (ch + 1 < nch) load(ch + 1, tid - 64, 192);
    } else if (lane < S) {
      const int rows = Ho - ch * R < R ? Ho - ch * R : R;
      const float *buf = tb + (ch & 1) * per + lane;
      const int n = rows * Tn;
      int it = 0;
      for (; it + 16 <= n; it += 16) {  // sixteen LDS reads in flight, then the sixteen dependent adds in order
        float t[16];
#pragma unroll
        for (int u = 0; u < 16; u++) t[u] = buf[(it + u) * S];
#pragma unroll
        for (int u = 0; u < 16; u++) cs = cs + t[u];
      }
      for (; it < n; it++) cs = cs + buf[it * S];
    }
    __syncthreads();
  }
  if (wave == 0 && lane < S) chsum[win * cs_ws + c0 + lane] = cs;
}

// fp32 channel sums, wave-private form (FORM 0 / 2, Wo <= 64): a wave owns 16 channels of one window and walks its
// image rows in order. Lane l loads the 16 channels' float4 quad (l & 3) of pixels 16 i + (l >> 2); 8 rows of those
// loads stay in flight in a register ring, so the wave keeps 8 x Wo x 64 bytes on the way (no LDS double buffer
// bounds it). A row that has landed goes through a wave-private LDS row [Wo][16], from which lanes 0..15 (one per
// channel) add the row's terms to their running sums in the reference's order: DW3 every pixel, DWK each 4-pixel
// group as (o0 + o1) + (o2 + o3), then the tail pixels. No block barrier: a wave's LDS writes and reads are in order.
template <int FORM, int NI>
__global__ __launch_bounds__(256) void k_chsum_w(const float *__restrict__ out, long long o_ws, int C, int Ho, int Wo,
                                                 float *__restrict__ chsum, long long cs_ws) {
  constexpr int NR = 8;  // rows in flight (the ring's loop is unrolled: longer rings land in scratch memory)
  __shared__ float rowb[4][64 * 16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, win = blockIdx.y;
  const int c0 = blockIdx.x * 64 + wave * 16;
  if (c0 >= C) return;
  const int nc = C - c0 < 16 ? C - c0 : 16;  // a multiple of 4
  const int p16 = lane >> 2, cq = lane & 3;
  // every lane loads (no branch, so the loads' counters stay exact and the ring stays in flight): rows past the image,
  // pixels past the row and quads past the channels read a valid address whose value no sum uses
  const float *img = out + win * o_ws + c0;  // wave-uniform
  int lofs[NI];                              // per lane: pixel 16 i + (l >> 2), quad (l & 3), in floats
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int px = 16 * i + p16;
    lofs[i] = (px < Wo ? px : Wo - 1) * C + 4 * (4 * cq < nc ? cq : 0);
  }
  float *rb = rowb[wave];
  float4 v[NR][NI];
  auto rowp = [&](int y) { return img + (long long)(y < Ho ? y : Ho - 1) * Wo * C; };  // wave-uniform
#pragma unroll
  for (int s = 0; s < NR; s++) {
    const float *rp = rowp(s);
#pragma unroll
    for (int i = 0; i < NI; i++)  // (the select keeps the compiler from placing the ring in scratch memory)
      v[s][i] = s < Ho ? *(const float4 *)(rp + lofs[i]) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int g4 = Wo & ~3;
  float cs = 0.f;
  for (int y0 = 0; y0 < Ho; y0 += NR) {
#pragma unroll
    for (int s = 0; s < NR; s++) {
      const int y = y0 + s;
      if (y >= Ho) break;
#pragma unroll
      for (int i = 0; i < NI; i++) *(float4 *)(rb + (16 * i + p16) * 16 + 4 * cq) = v[s][i];  // px < 64: in the row
      {  // the ring slot's next row
        const float *rp = rowp(y + NR);
#pragma unroll
        for (int i = 0; i < NI; i++) v[s][i] = *(const float4 *)(rp + lofs[i]);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (NI < 4 && lane < nc) {  // rows of at most 32 pixels: 16 LDS reads in flight, then their adds in order
        const float *col = rb + lane;
        if (FORM == 2) {
          int x = 0;
          for (; x + 16 <= Wo; x += 16) {
            float t[16];
#pragma unroll
            for (int u = 0; u < 16; u++) t[u] = col[(x + u) * 16];
#pragma unroll
            for (int u = 0; u < 16; u++) cs = cs + t[u];
          }
          for (; x < Wo; x++) cs = cs + col[x * 16];
        } else {
          for (int x = 0; x < g4; x += 4) {
            const float a = col[x * 16], b = col[(x + 1) * 16], c2 = col[(x + 2) * 16], d = col[(x + 3) * 16];
            cs = cs + ((a + b) + (c2 + d));
          }
          for (int x = g4; x < Wo; x++) cs = cs + col[x * 16];
        }
      }
      if (NI == 4 && lane < nc) {
        // rows of up to 64 pixels (the widest images, fewest waves): all the row's terms read from LDS at once (one
        // LDS round trip per row; 238 -> 193 us for 40 channels of 249 x 63 pixels), then added in order; reads past
        // the row's Wo pixels stay inside the wave's LDS row and are not used
        const float *col = rb + lane;
        float t[16 * NI];
#pragma unroll
        for (int u = 0; u < 16 * NI; u++) t[u] = col[u * 16];
        if (FORM == 2) {
#pragma unroll
          for (int u = 0; u < 16 * NI; u++)
            if (u < Wo) cs = cs + t[u];
        } else {
#pragma unroll
          for (int u = 0; u < 16 * NI; u += 4)
            if (u + 4 <= g4) cs = cs + ((t[u] + t[u + 1]) + (t[u + 2] + t[u + 3]));
#pragma unroll
          for (int u = 0; u < 16 * NI; u++)
            if (u >= g4 && u < Wo) cs = cs + t[u];
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
  if (lane < nc) chsum[win * cs_ws + c0 + lane] = cs;
}

// rows per chunk: two buffers of at most `cap` floats
static int chsum_rows(int Tn, int S, int Ho, int cap) {
  int R = cap / (Tn * S);
  if (R < 1) R = 1;
  return R < Ho ? R : Ho;
}

// one thread per (window, channel) walking the whole image: for channel counts that are not a multiple of 4
__global__ void k_chsum1_f32(const float *__restrict__ out, long long o_ws, int C, int Ho, int Wo, int form,
                            float *__restrict__ chsum, long long cs_ws, int B) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)B * C) return;
  const int win = (int)(i / C), c = (int)(i % C);
  const float *o = out + win * o_ws + c;
  float cs = 0.f;
  const int g4 = form == 0 ? (Wo & ~3) : 0;
  for (int oy = 0; oy < Ho; oy++) {
    const float *row = o + (long long)oy * Wo * C;
    for (int ox = 0; ox < g4; ox += 4) {
      const float s01 = row[(long long)ox * C] + row[(long long)(ox + 1) * C];
      const float s23 = row[(long long)(ox + 2) * C] + row[(long long)(ox + 3) * C];
      cs = cs + (s01 + s23);
    }
    for (int ox = g4; ox < Wo; ox++) cs = cs + row[(long long)ox * C];
  }
  chsum[win * cs_ws + c] = cs;
}
__global__ void k_chsum1_f16(const h16 *__restrict__ out, long long o_ws, int C, int Ho, int Wo, int form,
                            float *__restrict__ chsum, long long cs_ws, int B) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)B * C) return;
  const int win = (int)(i / C), c = (int)(i % C);
  const h16 *o = out + win * o_ws + c;
  float cs = 0.f;
  const int g4 = Wo & ~3, g2 = g4 + ((Wo - g4) & 2);
  for (int oy = 0; oy < Ho; oy++) {
    const h16 *row = o + (long long)oy * Wo * C;
    if (form == 3) {
      h16 rs = (h16)0.0f;
      for (int ox = 0; ox < Wo; ox++) rs = rs + row[(long long)ox * C];
      cs = cs + (float)rs;
      continue;
    }
    for (int ox = 0; ox < g4; ox += 4) {
      const h16 s = (row[(long long)ox * C] + row[(long long)(ox + 1) * C]) +
                    (row[(long long)(ox + 2) * C] + row[(long long)(ox + 3) * C]);
      cs = cs + (float)s;
    }
    if (g2 > g4) cs = cs + (float)(row[(long long)g4 * C] + row[(long long)(g4 + 1) * C]);
    if (Wo > g2) cs = cs + (float)row[(long long)g2 * C];
  }
  chsum[win * cs_ws + c] = cs;
}

template <typename T, int FORM>
static int chsum_launch(const T *out, long long o_ws, int C, int Ho, int Wo, float *chsum, long long cs_ws, int B,
                        hipStream_t st) {
  const int Tn = FORM == 0 ? Wo / 4 + Wo % 4 : FORM == 2 ? Wo : FORM == 1 ? Wo / 4 + ((Wo % 4) >> 1) + (Wo & 1) : 1;
  const int S = C < 64 ? C : 64;
  if (C % 4 || ((uintptr_t)out & (4 * sizeof(T) - 1)) || (B > 1 && o_ws % 4) || Tn * S > 8192) {
    if (sizeof(T) == 4)
      hipLaunchKernelGGL(k_chsum1_f32, dim3((unsigned)bnh_ceil_div((long long)B * C, 256)), dim3(256), 0, st,
                         (const float *)out, o_ws, C, Ho, Wo, FORM, chsum, cs_ws, B);
    else
      hipLaunchKernelGGL(k_chsum1_f16, dim3((unsigned)bnh_ceil_div((long long)B * C, 256)), dim3(256), 0, st,
                         (const h16 *)out, o_ws, C, Ho, Wo, FORM, chsum, cs_ws, B);
    BNH_HIP(hipGetLastError());
    return 0;
  }
  // fp32 sums over rows of at most 64 pixels: the wave-private form, from 33 channels up (with fewer, two waves per
  // window keep too little in flight: 24 channels of 249 x 63 pixels take about 177 us there against 166 us below)
  if constexpr (sizeof(T) == 4 && (FORM == 0 || FORM == 2)) {
    if (Wo <= 64 && C > 32) {
      const dim3 grid((unsigned)bnh_ceil_div(C, 64), (unsigned)B);
      const float *o = (const float *)out;
      if (Wo <= 16) hipLaunchKernelGGL((k_chsum_w<FORM, 1>), grid, dim3(256), 0, st, o, o_ws, C, Ho, Wo, chsum, cs_ws);
      else if (Wo <= 32) hipLaunchKernelGGL((k_chsum_w<FORM, 2>), grid, dim3(256), 0, st, o, o_ws, C, Ho, Wo, chsum, cs_ws);
      else hipLaunchKernelGGL((k_chsum_w<FORM, 4>), grid, dim3(256), 0, st, o, o_ws, C, Ho, Wo, chsum, cs_ws);
      BNH_HIP(hipGetLastError());
      return 0;
    }
  }
  // a block's chunk is one memory round trip of its loading waves: with at most one block per CU (no more blocks
  // than 2 per CU in the launch) the chunks take up to 144 KB of LDS, else 64 KB so that several blocks share a CU
  const long long nblk = bnh_ceil_div(C, 64) * (long long)B;
  const int cap = nblk <= 512 ? 18432 : 8192;
  const int R = chsum_rows(Tn, S, Ho, cap);
  const size_t lds = 2 * sizeof(float) * (size_t)R * Tn * S;
  if (lds > 64 * 1024)
    BNH_HIP(hipFuncSetAttribute((const void *)k_chsum<T, FORM>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  hipLaunchKernelGGL((k_chsum<T, FORM>), dim3((unsigned)bnh_ceil_div(C, 64), (unsigned)B), dim3(256), lds, st, out,
                     o_ws, C, Ho, Wo, R, chsum, cs_ws);
  BNH_HIP(hipGetLastError());
  return 0;
}

// ------------------------------------------------------------------ int8 depthwise (own specification)
// A thread owns 4 channels (one 32-bit word of every pixel) of a strip of NP consecutive output pixels of one row,
// numbered like the float kernels (window, row, strip, channel quad; XCD-contiguous blocks). Taps outside the image
// read the zero point, so that w (x - zx) vanishes there and
//   acc = bias - zx sum_t w[t] + sum_t w[t] x[t]   (mod 2^32, the specification's wrapping sum)
// holds for every output. Per input row the thread loads the strip's columns once, transposes each 4 columns x 4
// channels block so that a word holds 4 consecutive columns of one channel, and takes each output's taps of that row
// as a byte-aligned window of two such words: one v_dot4 per 4 taps, the row's taps packed the same way (zero past
// k). Loads and stores are buffer instructions: a per-lane 32-bit offset for the row plus a scalar column offset, so
// a strip inside the image spends no vector instruction on addresses; a strip at the left or right edge (EDGE)
// clamps its column offsets and selects the zero point outside. The activation table (LUT) sits in LDS.
// output pixels per thread: 8 at stride 1 (the setup, the taps and the transposes shared by more outputs), 4 at 2
__host__ __device__ constexpr int dw_s8_np(int s) { return s == 1 ? 8 : 4; }
template <int K, int S, bool EDGE>
BNH_DEV void dw_s8_strip(__amdgpu_buffer_rsrc_t xr, int x_off, int ix0, int H, int W, int C, int iy0, uint32_t zxw,
                         const uint32_t (&wp)[K][(K + 3) / 4][4], int32_t (&acc)[dw_s8_np(S)][4]) {
  constexpr int NP = dw_s8_np(S), NG = (K + 3) / 4, NCOL = (NP - 1) * S + K;
  constexpr int ND = ((NP - 1) * S + 4 * (NG - 1)) / 4 + 2;  // 4-column words per channel and row
  int coff[NCOL];
  bool cok[NCOL];
#pragma unroll
  for (int col = 0; col < NCOL; col++) {
    const int ix = ix0 + col;
    cok[col] = (unsigned)ix < (unsigned)W;
    coff[col] = (ix < 0 ? 0 : ix >= W ? W - 1 : ix) * C;
  }
#pragma unroll
  for (int ky = 0; ky < K; ky++) {
    const int iy = iy0 + ky;
    uint32_t r[4 * ND];
#pragma unroll
    for (int col = 0; col < 4 * ND; col++) r[col] = col < NCOL ? zxw : 0u;
    if ((unsigned)iy < (unsigned)H) {
      const int ro = x_off + iy * W * C;
#pragma unroll
      for (int col = 0; col < NCOL; col++) {
        if (EDGE) {
          const uint32_t v = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(xr, ro + coff[col], 0, 0);
          r[col] = cok[col] ? v : zxw;
        } else {  // the lane's first column in the vector offset, the column step in the scalar one
          r[col] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(xr, ro + ix0 * C, col * C, 0);
        }
      }
    }
    uint32_t d[ND][4];  // d[j][ch]: columns 4j..4j+3 of channel ch
#pragma unroll
    for (int j = 0; j < ND; j++) transpose4x4(r[4 * j], r[4 * j + 1], r[4 * j + 2], r[4 * j + 3], d[j]);
#pragma unroll
    for (int q = 0; q < NP; q++)
#pragma unroll
      for (int j = 0; j < NG; j++) {
        const int o = q * S + 4 * j, b = o >> 2, sh = o & 3;
#pragma unroll
        for (int ch = 0; ch < 4; ch++) {
          const uint32_t v = sh ? __builtin_amdgcn_alignbyte(d[b + 1][ch], d[b][ch], sh) : d[b][ch];
          acc[q][ch] = __builtin_amdgcn_sdot4((int)v, (int)wp[ky][j][ch], acc[q][ch], false);
        }
      }
  }
}

template <int K, int S, bool LUT>
__global__ __launch_bounds__(256) void k_dw_s8(const int8_t *__restrict__ x, long long x_ws, unsigned x_len, int H,
                                               int W, int C, int pt, int pl, const int8_t *__restrict__ w,
                                               const int32_t *__restrict__ bias, const int32_t *__restrict__ mult,
                                               const int32_t *__restrict__ shift, int zx, int zy, int lo, int hi,
                                               const int8_t *__restrict__ lut, int8_t *__restrict__ out,
                                               long long o_ws, unsigned o_len, int Ho, int Wo, long long total,
                                               DwGrid g) {
  constexpr int NP = dw_s8_np(S), NG = (K + 3) / 4, NCOL = (NP - 1) * S + K;
  __shared__ int8_t s_lut[256];
  if (LUT) {
    s_lut[threadIdx.x] = lut[threadIdx.x];
    __syncthreads();
  }
  const DwPos ps = dw_pos(C >> 2, Ho, total, g);
  if (!ps.ok) return;
  const int c = ps.c * 4, oy = ps.oy, px0 = ps.it0;
  const uint32_t zxw = (uint32_t)(uint8_t)zx * 0x01010101u;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void *)w, 0, K * K * C, 0x00020000);
  // the taps, per row ky, group j and channel ch: bytes w[ky][4j + 0..3][c + ch]
  uint32_t wp[K][NG][4];
  uint32_t wsum[4] = {0, 0, 0, 0};
#pragma unroll
  for (int ky = 0; ky < K; ky++)
#pragma unroll
    for (int j = 0; j < NG; j++) {
      uint32_t r[4];
#pragma unroll
      for (int i = 0; i < 4; i++)
        r[i] = 4 * j + i < K ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(wr, c, (ky * K + 4 * j + i) * C, 0) : 0u;
      transpose4x4(r[0], r[1], r[2], r[3], wp[ky][j]);
#pragma unroll
      for (int ch = 0; ch < 4; ch++)
        wsum[ch] = (uint32_t)__builtin_amdgcn_sdot4((int)wp[ky][j][ch], 0x01010101, (int)wsum[ch], false);
    }
  int32_t acc[NP][4];
  // the short requantisation (below) needs sums that cannot wrap: |bias - zx sum w| + K^2 2^14 < 2^31
  bool nowrap = true;
#pragma unroll
  for (int ch = 0; ch < 4; ch++) {
    const int32_t a0 = (int32_t)((uint32_t)bias[c + ch] - (uint32_t)zx * wsum[ch]);
    nowrap = nowrap && (a0 < 0 ? -(long long)a0 : (long long)a0) + (long long)K * K * 16384 < (1LL << 31);
#pragma unroll
    for (int q = 0; q < NP; q++) acc[q][ch] = a0;
  }
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void *)x, 0, (int)x_len, 0x00020000);
  const int x_off = (int)(ps.win * x_ws) + c, ix0 = px0 * S - pl, iy0 = oy * S - pt;
  if (ix0 < 0 || ix0 + NCOL > W) dw_s8_strip<K, S, true>(xr, x_off, ix0, H, W, C, iy0, zxw, wp, acc);
  else dw_s8_strip<K, S, false>(xr, x_off, ix0, H, W, C, iy0, zxw, wp, acc);
  int32_t m[4], e[4];
  bool s1 = true;  // every shift of the thread's channels in 1..31: the one-rounding requant
#pragma unroll
  for (int ch = 0; ch < 4; ch++) {
    m[ch] = mult[c + ch];
    e[ch] = shift[c + ch];
    s1 = s1 && e[ch] >= 1 && e[ch] <= 31;
  }
  const __amdgpu_buffer_rsrc_t orr = __builtin_amdgcn_make_buffer_rsrc((void *)out, 0, (int)o_len, 0x00020000);
  const int o_off = (int)(ps.win * o_ws) + (oy * Wo + px0) * C + c;
  auto store = [&](auto requant) {
#pragma unroll
    for (int q = 0; q < NP; q++) {
      if (px0 + q >= Wo) break;
      uint32_t word = 0;
#pragma unroll
      for (int ch = 0; ch < 4; ch++) {
        int32_t y = requant(acc[q][ch], ch);
        if (LUT) y = s_lut[y + 128];
        word |= ((uint32_t)y & 0xffu) << (8 * ch);
      }
      __builtin_amdgcn_raw_buffer_store_b32(word, orr, o_off, q * C, 0);
    }
  };
  if (s1 && nowrap && zy <= lo) {
    // zy <= lo: a negative product requantises to lo under either rounding of its sign, so the one-rounding form
    // needs no sign test and the zero point moves outside the clamp: zy + clamp(hi32(acc m + 2^30 + 2^(30+e)) >> (e-1),
    // lo - zy, hi - zy) (|acc m| < 2^62: the shifted value is far from int32's ends, so the saturating add never
    // saturates)
    long long a0[4];
    int e1[4];
#pragma unroll
    for (int ch = 0; ch < 4; ch++) {
      a0[ch] = (1LL << 30) + (1LL << (30 + e[ch]));
      e1[ch] = e[ch] - 1;
    }
    const int lz = lo - zy, hz = hi - zy;
    store([&](int32_t a, int ch) {
      const int32_t v = (int32_t)(((long long)a * m[ch] + a0[ch]) >> 32) >> e1[ch];
      int32_t cl;
      asm("v_med3_i32 %0, %1, %2, %3" : "=v"(cl) : "v"(v), "v"(lz), "v"(hz));
      return cl + zy;
    });
  } else if (s1) {
    BnhRqS1 rc[4];
#pragma unroll
    for (int ch = 0; ch < 4; ch++) rc[ch] = bnh_rq_s1(e[ch]);
    store([&](int32_t a, int ch) { return bnh_requant_s1(a, m[ch], rc[ch], zy, lo, hi); });
  } else {
    store([&](int32_t a, int ch) { return bnh_requant(a, m[ch], e[ch], zy, lo, hi); });
  }
}

// ------------------------------------------------------------------ int8 depthwise, stride 1, row-streamed
// A block computes 32 channels x 64 output columns of one window over a segment of output rows, 4 rows a step, with
// the input rows it needs in an LDS ring of 8 row slots (blocks numbered channel group fastest, then column tile,
// segment and window, XCD-contiguous, so that the blocks reading the same pixels' other channels share an L2). In
// the ring each input row is held as planes of one channel, a word holding 4 consecutive columns, written from
// 16-byte loads (4 columns x 16 channels) transposed 4 x 4 in registers; pixels outside the image (and channels
// past C) hold the zero point, so that w (x - zx) vanishes there and acc = bias - zx sum_t w[t] + sum_t w[t] x[t]
// (mod 2^32) holds for every output, as in k_dw_s8. A thread owns one channel and 8 consecutive output columns: per
// tap row it reads the 3 words covering its 8 + K - 1 input columns, and output column 4h + r of its 8 takes its K
// taps as v_dot4 of words h and h + 1 with the row's weights shifted by r bytes (prepared once per thread for the
// four shifts), so no byte realignment is done per tap. While a step computes, the loads of the next step's 4 input
// rows are in flight in registers; they go into the ring slots of the 4 rows the step no longer needs after it.
// The requantised bytes go through LDS planes, are transposed back to 4-channel words and stored as 16 bytes.
constexpr int kDwtStep = 4, kDwtSeg = 12;
template <int K, int CT, int TW>
struct DwtShape {
  static constexpr int NG = CT / 16;                    // 16-channel groups
  static constexpr int NR = kDwtStep + K - 1;           // input rows a step reads
  static constexpr int IW = (TW + K - 1 + 3) / 4;       // input words per row and channel
  static constexpr int PI = (8 * IW) | 1;               // words per channel plane of the 8-slot ring (odd: the 32
                                                        // channels' reads of one word fall in 32 banks)
  static constexpr int OW = TW / 4;                     // output words per row
  static constexpr int PO = (kDwtStep * OW) | 1;
  static_assert(NR <= 8, "a step's input rows fit the ring");
};

template <int K, int CT, int TW, bool LUT>
__global__ __launch_bounds__(256) void k_dw_s8_t(const int8_t *__restrict__ x, long long x_ws, unsigned x_len, int H,
                                                 int W, int C, int pt, int pl, const int8_t *__restrict__ w,
                                                 const int32_t *__restrict__ bias, const int32_t *__restrict__ mult,
                                                 const int32_t *__restrict__ shift, int zx, int zy, int lo, int hi,
                                                 const int8_t *__restrict__ lut, int8_t *__restrict__ out,
                                                 long long o_ws, unsigned o_len, int Ho, int Wo, int ncg, int ntx,
                                                 int nseg) {
  using S = DwtShape<K, CT, TW>;
  static_assert(CT * TW / 8 == 256, "a thread per channel and 8 columns");
  __shared__ uint32_t s_in[CT * S::PI];
  __shared__ uint32_t s_out[CT * S::PO];
  __shared__ int8_t s_lut[256];
  const int tid = threadIdx.x;
  if (LUT) s_lut[tid] = lut[tid];
  unsigned L = bnh_xcd_block(blockIdx.x, gridDim.x);
  const int cg = (int)(L % (unsigned)ncg);
  L /= (unsigned)ncg;
  const int tx = (int)(L % (unsigned)ntx);
  L /= (unsigned)ntx;
  const int sg = (int)(L % (unsigned)nseg);
  const int win = (int)(L / (unsigned)nseg);
  const int c0 = cg * CT, ox0 = tx * TW, oy0 = sg * kDwtSeg, ix0 = ox0 - pl, iy0 = oy0 - pt;
  const int nstep = (min(kDwtSeg, Ho - oy0) + kDwtStep - 1) / kDwtStep;
  const uint32_t zxw = (uint32_t)(uint8_t)zx * 0x01010101u;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void *)x, 0, (int)x_len, 0x00020000);
  const int xw = (int)(win * x_ws);
  // unit u of a set of input rows = (row of the set, word wd, 16-channel group g), g fastest: 4 columns x 16
  // channels as four 16-byte loads (the zero point outside the image and for channels past C)
  auto load_unit = [&](int u, int r0, v4i (&v)[4]) {
    const int g = u % S::NG, p = u / S::NG, rr = p / S::IW, wd = p - rr * S::IW;
    const int iy = iy0 + r0 + rr, ixb = ix0 + 4 * wd, c = c0 + 16 * g;
    const bool rok = (unsigned)iy < (unsigned)H;
    const int ro = xw + iy * W * C + c;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int ix = ixb + i;
      if (rok && (unsigned)ix < (unsigned)W) {
        v[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, ro + ix * C, 0, 0);
#pragma unroll
        for (int j = 0; j < 4; j++)
          if (c + 4 * j >= C) v[i][j] = (int)zxw;
      } else {
        v[i] = v4i{(int)zxw, (int)zxw, (int)zxw, (int)zxw};
      }
    }
  };
  // ... and its four 4 x 4 transposes into the ring: word wd of row r0 + rr's slot in planes 16g .. 16g + 15
  auto put_unit = [&](int u, int r0, const v4i (&v)[4]) {
    const int g = u % S::NG, p = u / S::NG, rr = p / S::IW, wd = p - rr * S::IW;
    const int at = ((r0 + rr) & 7) * S::IW + wd;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint32_t t[4];
      transpose4x4((uint32_t)v[0][j], (uint32_t)v[1][j], (uint32_t)v[2][j], (uint32_t)v[3][j], t);  // t[i]: channel
#pragma unroll                                                                                     // c + 4j + i
      for (int i = 0; i < 4; i++) s_in[(16 * g + 4 * j + i) * S::PI + at] = t[i];
    }
  };
  // the first step's input rows
  for (int u = tid; u < S::NR * S::IW * S::NG; u += 256) {
    v4i v[4];
    load_unit(u, 0, v);
    put_unit(u, 0, v);
  }
  // the thread's channel, its weights per tap row and shift, and its requantisation
  const int ch = tid % CT, sub = tid / CT, c = c0 + ch;
  const bool cok = c < C;
  // ws[ky][r][h]: byte p = w[ky][4h + p - r] (0 where that tap index is outside 0..K-1), from the row's taps packed
  // into two words (w0..w3, w4..w7 with zeros past K): word 0 is the first shifted up by r bytes, word 1 the pair
  // shifted by r bytes across the word boundary
  uint32_t ws[K][4][2];
  uint32_t wsum = 0;
#pragma unroll
  for (int ky = 0; ky < K; ky++) {
    uint32_t W0 = 0, W1 = 0;
#pragma unroll
    for (int kx = 0; kx < K; kx++) {
      const int32_t v = cok ? (int32_t)w[(ky * K + kx) * C + c] : 0;
      wsum += (uint32_t)v;
      if (kx < 4) W0 |= ((uint32_t)v & 0xffu) << (8 * kx);
      else W1 |= ((uint32_t)v & 0xffu) << (8 * (kx - 4));
    }
    ws[ky][0][0] = W0;
    ws[ky][0][1] = W1;
#pragma unroll
    for (int r = 1; r < 4; r++) {
      ws[ky][r][0] = W0 << (8 * r);
      ws[ky][r][1] = __builtin_amdgcn_alignbyte(W1, W0, 4 - r);
    }
  }
  const int32_t a0 = cok ? (int32_t)((uint32_t)bias[c] - (uint32_t)zx * wsum) : 0;
  const int32_t m = cok ? mult[c] : 0, e = cok ? shift[c] : 1;
  const bool nowrap = (a0 < 0 ? -(long long)a0 : (long long)a0) + (long long)K * K * 16384 < (1LL << 31);
  // the short requantisation of k_dw_s8 (shift in 1..31, sums that cannot wrap, zy <= lo) when the whole wave
  // qualifies, else the general one
  const bool fast = __all(e >= 1 && e <= 31 && nowrap && zy <= lo);
  const long long rnd = (1LL << 30) + (1LL << (30 + (fast ? e : 1)));
  const int e1 = fast ? e - 1 : 0, lz = lo - zy, hz = hi - zy, zy128 = zy + 128;
  const __amdgpu_buffer_rsrc_t orr = __builtin_amdgcn_make_buffer_rsrc((void *)out, 0, (int)o_len, 0x00020000);
  const int ow = (int)(win * o_ws);
  __syncthreads();
  // one step: output rows oy0 + 4 st .. + 3 from ring rows 4 st .. 4 st + NR - 1; FAST picks the requantisation,
  // B = (4 st) & 7 the ring slot of the step's first input row
  auto step = [&]<bool FAST, int B>(int st) {
    auto requant = [&](int32_t a) -> uint32_t {
      int32_t y;
      if (FAST) {
        const int32_t v = (int32_t)(((long long)a * m + rnd) >> 32) >> e1;
        asm("v_med3_i32 %0, %1, %2, %3" : "=v"(y) : "v"(v), "v"(lz), "v"(hz));
        if (LUT) return (uint32_t)(uint8_t)s_lut[y + zy128];  // the table at y + zy
        y += zy;
      } else {
        y = bnh_requant(a, m, e, zy, lo, hi);
        if (LUT) y = s_lut[y + 128];
      }
      return (uint32_t)y & 0xffu;
    };
    // the next step's 4 new input rows (ring rows 4 st + NR ..), in flight while this step computes
    const bool more = st + 1 < nstep;
    constexpr int NPF = kDwtStep * S::IW * S::NG, PFI = (NPF + 255) / 256;  // units of the 4 rows, per thread
    const int r_next = 4 * st + S::NR;
    v4i pv[PFI][4];
#pragma unroll
    for (int i = 0; i < PFI; i++)
      if (more && tid + 256 * i < NPF) load_unit(tid + 256 * i, r_next, pv[i]);
    uint32_t res[kDwtStep][2];
    const uint32_t *plane = s_in + ch * S::PI + 2 * sub;
#pragma unroll
    for (int oy = 0; oy < kDwtStep; oy++) {
      int32_t acc[8];
#pragma unroll
      for (int q = 0; q < 8; q++) acc[q] = a0;
#pragma unroll
      for (int ky = 0; ky < K; ky++) {
        const uint32_t *row = plane + ((B + oy + ky) & 7) * S::IW;
        const uint32_t A[3] = {row[0], row[1], row[2]};
#pragma unroll
        for (int q = 0; q < 8; q++) {
          const int h = q >> 2, r = q & 3;
          acc[q] = __builtin_amdgcn_sdot4((int)A[h], (int)ws[ky][r][0], acc[q], false);
          if (r >= 5 - K) acc[q] = __builtin_amdgcn_sdot4((int)A[h + 1], (int)ws[ky][r][1], acc[q], false);
        }
      }
#pragma unroll
      for (int h = 0; h < 2; h++)
        res[oy][h] = requant(acc[4 * h]) | requant(acc[4 * h + 1]) << 8 | requant(acc[4 * h + 2]) << 16 |
                     requant(acc[4 * h + 3]) << 24;
    }
    __syncthreads();  // the step's reads of the ring and the previous step's reads of s_out are done
#pragma unroll
    for (int oy = 0; oy < kDwtStep; oy++)
#pragma unroll
      for (int h = 0; h < 2; h++) s_out[ch * S::PO + oy * S::OW + 2 * sub + h] = res[oy][h];
#pragma unroll
    for (int i = 0; i < PFI; i++)
      if (more && tid + 256 * i < NPF) put_unit(tid + 256 * i, r_next, pv[i]);
    __syncthreads();
    // store: unit = (output row, word wd, 16-channel group g), g fastest: sixteen plane words, four transposes back,
    // four 16-byte stores (word by word for a group that reaches past C)
    for (int u = tid; u < kDwtStep * S::OW * S::NG; u += 256) {
      const int g = u % S::NG, p = u / S::NG, oy = p / S::OW, wd = p - oy * S::OW;
      const int y = oy0 + 4 * st + oy, cq = c0 + 16 * g;
      if (y < Ho && cq < C) {
        v4i v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          uint32_t t[4], o4[4];
#pragma unroll
          for (int i = 0; i < 4; i++) t[i] = s_out[(16 * g + 4 * j + i) * S::PO + p];
          transpose4x4(t[0], t[1], t[2], t[3], o4);  // o4[col]: the column's channels cq + 4j .. + 3
#pragma unroll
          for (int col = 0; col < 4; col++) v[col][j] = (int)o4[col];
        }
        const int o = ow + (y * Wo + ox0 + 4 * wd) * C + cq;
        const bool whole = cq + 16 <= C;
#pragma unroll
        for (int col = 0; col < 4; col++) {
          if (ox0 + 4 * wd + col >= Wo) break;
          if (whole) {
            __builtin_amdgcn_raw_buffer_store_b128(v[col], orr, o + col * C, 0, 0);
          } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
              if (cq + 4 * j < C) __builtin_amdgcn_raw_buffer_store_b32(v[col][j], orr, o + col * C + 4 * j, 0, 0);
          }
        }
      }
    }
  };
  for (int st = 0; st < nstep; st++) {
    if (fast) {
      if (st & 1) step.template operator()<true, 4>(st);
      else step.template operator()<true, 0>(st);
    } else {
      if (st & 1) step.template operator()<false, 4>(st);
      else step.template operator()<false, 0>(st);
    }
  }
}

// ================================================================== host side
template <typename T, typename L>
static void dispatch_ks(int k, int s, L &&launch) {
  if (k == 1 && s == 1) launch.template operator()<1, 1>();
  else if (k == 1 && s == 2) launch.template operator()<1, 2>();
  else if (k == 3 && s == 1) launch.template operator()<3, 1>();
  else if (k == 3 && s == 2) launch.template operator()<3, 2>();
  else if (k == 5 && s == 1) launch.template operator()<5, 1>();
  else if (k == 5 && s == 2) launch.template operator()<5, 2>();
  else if (k == 7 && s == 1) launch.template operator()<7, 1>();
  else launch.template operator()<7, 2>();
}

// the fp16 kernels run channel pairs when every pair is 4-byte aligned
static bool dw_pairs(const void *xp, long long x_ws, const void *w, const void *b, const void *out, long long o_ws, int C,
                     int B) {
  return C % 2 == 0 && ((uintptr_t)xp & 3) == 0 && ((uintptr_t)w & 3) == 0 && ((uintptr_t)b & 3) == 0 &&
         ((uintptr_t)out & 3) == 0 && (B == 1 || (x_ws % 2 == 0 && o_ws % 2 == 0));
}

// the fp16 kernels run channel quads when every quad is 8-byte aligned and the batch's input and output each stay
// under 2 GiB (32-bit buffer offsets); px_in / px_out: pixels per window (haloed input)
static bool dw_quads(const void *xp, long long x_ws, const void *w, const void *b, const void *out, long long o_ws,
                     int C, int B, long long px_in, long long px_out) {
  return C % 4 == 0 && ((uintptr_t)xp & 7) == 0 && ((uintptr_t)w & 7) == 0 && ((uintptr_t)b & 7) == 0 &&
         ((uintptr_t)out & 7) == 0 && (B == 1 || (x_ws % 4 == 0 && o_ws % 4 == 0)) &&
         2 * ((long long)(B - 1) * x_ws + px_in * C) < (1LL << 31) &&
         2 * ((long long)(B - 1) * o_ws + px_out * C) < (1LL << 31) && 2LL * 49 * C < (1LL << 31);
}

static int dw_check(int H, int W, int C, int k, int s, int pt, int pl, int Ho, int Wo, int B, long long x_ws,
                    long long o_ws, int halo) {
  BNH_REQ(H > 0 && W > 0 && C > 0 && Ho > 0 && Wo > 0 && B > 0);
  BNH_REQ(k == 1 || k == 3 || k == 5 || k == 7);
  BNH_REQ(s == 1 || s == 2);
  const int h = halo;
  BNH_REQ(pt >= 0 && pt <= h && pl >= 0 && pl <= h);
  BNH_REQ((Ho - 1) * s - pt + k <= H + h && (Wo - 1) * s - pl + k <= W + h);  // the last tap stays in the halo
  BNH_REQ(B == 1 || (x_ws >= (long long)(H + 2 * h) * (W + 2 * h) * C && o_ws >= (long long)Ho * Wo * C));
  BNH_REQ((long long)B * Ho * Wo * C / 256 < (1LL << 31));
  return 0;
}

// the fused kernel's plan: KS K steps per MFMA tile (a power of two: the weight fragments a lane holds), TH output
// rows per band (nband bands of at most TH rows), gsplit blocks per band (parts of the channel groups), LDS rows of WL
// padded columns at a stride of RS floats, the per-pixel arrays at float offset sz_off (npx pixels each), lds bytes
// per block
struct PwdwPlan {
  int KS, TH, nband, gsplit, WL, RS, sz_off, npx;
  size_t lds;
};
static int pwdw_plan(int C, int Kp, int H, int W, int k, int s, int pt, int pl, int form, int Ho, int Wo, int B,
                     PwdwPlan *pp) {
  BNH_REQ(C > 0 && C % 16 == 0 && Kp > 0 && Kp % 16 == 0);
  BNH_REQ((k == 3 || k == 5) && (s == 1 || s == 2));
  BNH_REQ(form == 0 || (form == 2 && k == 3 && pt == 1 && pl == 1));
  const int h = (k - 1) / 2;
  BNH_REQ(H > 0 && W > 0 && Ho > 0 && Wo > 0 && pt >= 0 && pt <= h && pl >= 0 && pl <= h);
  BNH_REQ((Ho - 1) * s - pt + k <= H + h && (Wo - 1) * s - pl + k <= W + h);  // the last tap stays in the halo
  BNH_REQ(Ho <= 65536 && (long long)Ho * items_per_row(Wo, form) < 65536);  // positions of a band (float indexing)
  if (Kp > 512) return bnh_fail("bnh_pwdw_f32: K %d: the fused kernel holds at most 512 int8 columns per row", Kp);
  int KS = 1;
  while (64 * KS < Kp) KS *= 2;
  const int WL = (Wo - 1) * s + k;
  int RS = WL * 20;
  while ((s * RS) % 64 != 16) RS += 4;
  // LDS per block: three blocks per CU (the kernel's registers allow no more)
  const long long budget = 52 * 1024;
  auto bytes = [&](int TH) {  // RIN rows of cells + discard cells, 12 bytes per pixel + its int8 row
    const long long rin = (long long)(TH - 1) * s + k, px = (rin * W + 15) / 16 * 16;
    return 4 * (rin * RS + 64) + px * (12 + Kp);
  };
  if (bytes(1) > budget)
    return bnh_fail("bnh_pwdw_f32: %d input columns (%d padded columns, K %d) leave no band of one output row in %lld "
                    "bytes of LDS", W, WL, Kp, budget);
  int TH = 1;
  while (TH < Ho && bytes(TH + 1) <= budget) TH++;
  const int nband = (Ho + TH - 1) / TH;
  TH = (Ho + nband - 1) / nband;  // bands of equal height
  // parts of the channel groups: enough blocks to fill the chip (about 2048), at least 2 groups per part
  const long long nb = (long long)B * nband;
  int gsplit = nb >= 2048 ? 1 : (int)bnh_ceil_div(2048, nb);
  if (gsplit > C / 32) gsplit = C / 32 > 1 ? C / 32 : 1;
  const long long rin = (long long)(TH - 1) * s + k;
  pp->KS = KS;
  pp->TH = TH;
  pp->nband = nband;
  pp->gsplit = gsplit;
  pp->WL = WL;
  pp->RS = RS;
  pp->sz_off = (int)(rin * RS + 64);
  pp->npx = (int)((rin * W + 15) / 16 * 16);
  pp->lds = (size_t)bytes(TH);
  return 0;
}

extern "C" {

int bnh_dwk_f32(const float *xp, long long x_ws, int H, int W, int C, int k, int s, int pt, int pl, const float *w,
                const float *b, int act, float *out, long long o_ws, int Ho, int Wo, float *chsum, long long cs_ws,
                int B, void *stream) {
  BNH_REQ(xp && w && b && out && (act == 0 || act == 1));
  if (dw_check(H, W, C, k, s, pt, pl, Ho, Wo, B, x_ws, o_ws, (k - 1) / 2)) return -1;
  const int nit = items_per_row(Wo, 0);
  unsigned nb;
  long long total;
  DwGrid g;
  if (dw_grid(nit, dw_ni(k), C, Ho, B, &nb, &total, &g)) return -1;
  hipStream_t st = bnh_stream(stream);
  const int Wp = W + k - 1;
  dispatch_ks<float>(k, s, [&]<int K, int S>() {
    hipLaunchKernelGGL((k_dw_f32<K, S, 0>), dim3(nb), dim3(256), 0, st, xp, x_ws, Wp, C, pt, pl, w, b, act, out, o_ws,
                       Ho, Wo, nit, total, g);
  });
  BNH_HIP(hipGetLastError());
  if (chsum) {
    BNH_REQ(B == 1 || cs_ws >= C);
    if (chsum_launch<float, 0>(out, o_ws, C, Ho, Wo, chsum, cs_ws, B, st)) return -1;
  }
  return 0;
}

int bnh_dw3_f32(const float *xp, long long x_ws, int H, int W, int C, int s, const float *w, const float *b, float *out,
                long long o_ws, int Ho, int Wo, float *chsum, long long cs_ws, int B, void *stream) {
  BNH_REQ(xp && w && b && out);
  if (dw_check(H, W, C, 3, s, 1, 1, Ho, Wo, B, x_ws, o_ws, 1)) return -1;
  const int nit = items_per_row(Wo, 2);
  unsigned nb;
  long long total;
  DwGrid g;
  if (dw_grid(nit, dw_ni(3), C, Ho, B, &nb, &total, &g)) return -1;
  hipStream_t st = bnh_stream(stream);
  // stride 1 on channel pairs (8-byte aligned, 32-bit buffer offsets): bands of R output rows
  constexpr int R = 6;
  const long long x_len = 4 * ((long long)(B - 1) * x_ws + (long long)(H + 2) * (W + 2) * C);
  const long long o_len = 4 * ((long long)(B - 1) * o_ws + (long long)Ho * Wo * C);
  if (s == 1 && C % 2 == 0 && ((uintptr_t)xp & 7) == 0 && ((uintptr_t)w & 7) == 0 && ((uintptr_t)b & 7) == 0 &&
      ((uintptr_t)out & 7) == 0 && (B == 1 || (x_ws % 2 == 0 && o_ws % 2 == 0)) &&
      x_len + 4LL * (R + 2) * (W + 2) * C < (1LL << 31) && o_len + 4LL * R * Wo * C < (1LL << 31)) {
    if (dw_grid(Wo, 4, C / 2, (Ho + R - 1) / R, B, &nb, &total, &g)) return -1;
    hipLaunchKernelGGL((k_dw3_f32v<1, R>), dim3(nb), dim3(256), 0, st, xp, x_ws, (unsigned)x_len, W + 2, C, w, b, out,
                       o_ws, (unsigned)o_len, Ho, Wo, total, g);
  } else if (s == 1)
    hipLaunchKernelGGL((k_dw_f32<3, 1, 2>), dim3(nb), dim3(256), 0, st, xp, x_ws, W + 2, C, 1, 1, w, b, 1, out, o_ws,
                       Ho, Wo, nit, total, g);
  else
    hipLaunchKernelGGL((k_dw_f32<3, 2, 2>), dim3(nb), dim3(256), 0, st, xp, x_ws, W + 2, C, 1, 1, w, b, 1, out, o_ws,
                       Ho, Wo, nit, total, g);
  BNH_HIP(hipGetLastError());
  if (chsum) {
    BNH_REQ(B == 1 || cs_ws >= C);
    if (chsum_launch<float, 2>(out, o_ws, C, Ho, Wo, chsum, cs_ws, B, st)) return -1;
  }
  return 0;
}

int bnh_pwdw_f32_plan(int C, int Kp, int H, int W, int k, int s, int pt, int pl, int form, int Ho, int Wo) {
  PwdwPlan pp;
  return pwdw_plan(C, Kp, H, W, k, s, pt, pl, form, Ho, Wo, 1, &pp);
}

int bnh_pwdw_f32(const int8_t *q, long long q_ws, const float *sa, long long sa_ws, const int32_t *za, long long za_ws,
                 int H, int W, const bnh_s8w *Wt, int pact, int k, int s, int pt, int pl, int form, const float *w,
                 const float *b, int dact, float *out, long long o_ws, int Ho, int Wo, float *chsum, long long cs_ws,
                 int B, void *stream) {
  BNH_REQ(q && sa && za && Wt && w && b && out && B > 0);
  BNH_REQ(pact >= 0 && pact <= 2 && (dact == 0 || dact == 1));
  const int C = Wt->Np, Kp = Wt->Kp;
  PwdwPlan pp;
  if (pwdw_plan(C, Kp, H, W, k, s, pt, pl, form, Ho, Wo, B, &pp)) return -1;
  const long long M = (long long)H * W;
  BNH_REQ(((uintptr_t)q & 15) == 0 && q_ws % 16 == 0);
  BNH_REQ(B == 1 || (q_ws >= M * Kp && sa_ws >= M && za_ws >= M && o_ws >= (long long)Ho * Wo * C));
  const long long nblk = (long long)B * pp.nband * pp.gsplit;
  BNH_REQ(nblk < (1LL << 31));
  const int nit = items_per_row(Wo, form);
  hipStream_t st = bnh_stream(stream);
#define PWDW(KK, SS, FF, KS_)                                                                                          \
  hipLaunchKernelGGL((k_pwdw_f32<KK, SS, FF, KS_>), dim3((unsigned)nblk), dim3(256), pp.lds, st, q, q_ws, sa, sa_ws, za, \
                     za_ws, H, W, Kp, Wt->w, Wt->sw, Wt->colsum, Wt->b, pact, C, pt, pl, w, b, dact, out, o_ws, Ho, Wo, \
                     nit, pp.TH, pp.nband, pp.gsplit, pp.WL, pp.RS, pp.sz_off, pp.npx, 1.0 / W)
#define PWDW_KS(KK, SS, FF)                                                                                            \
  do {                                                                                                                 \
    if (pp.KS == 1) PWDW(KK, SS, FF, 1);                                                                               \
    else if (pp.KS == 2) PWDW(KK, SS, FF, 2);                                                                          \
    else if (pp.KS == 4) PWDW(KK, SS, FF, 4);                                                                          \
    else PWDW(KK, SS, FF, 8);                                                                                          \
  } while (0)
  if (form == 2) {
    if (s == 1) PWDW_KS(3, 1, 2);
    else PWDW_KS(3, 2, 2);
  } else if (k == 3) {
    if (s == 1) PWDW_KS(3, 1, 0);
    else PWDW_KS(3, 2, 0);
  } else {
    if (s == 1) PWDW_KS(5, 1, 0);
    else PWDW_KS(5, 2, 0);
  }
#undef PWDW_KS
#undef PWDW
  BNH_HIP(hipGetLastError());
  if (chsum) {
    BNH_REQ(B == 1 || cs_ws >= C);
    if (form == 2 ? chsum_launch<float, 2>(out, o_ws, C, Ho, Wo, chsum, cs_ws, B, st)
                  : chsum_launch<float, 0>(out, o_ws, C, Ho, Wo, chsum, cs_ws, B, st))
      return -1;
  }
  return 0;
}

int bnh_dwk_f16(const uint16_t *xp, long long x_ws, int H, int W, int C, int k, int s, int pt, int pl,
                const uint16_t *w, const uint16_t *b, int act, uint16_t *out, long long o_ws, int Ho, int Wo,
                float *chsum, long long cs_ws, int B, void *stream) {
  BNH_REQ(xp && w && b && out && (act == 0 || act == 1));
  if (dw_check(H, W, C, k, s, pt, pl, Ho, Wo, B, x_ws, o_ws, (k - 1) / 2)) return -1;
  const int nit = items_per_row(Wo, 1);
  unsigned nb;
  long long total;
  DwGrid g;
  hipStream_t st = bnh_stream(stream);
  const int Wp = W + k - 1;
  if (dw_quads(xp, x_ws, w, b, out, o_ws, C, B, (long long)(H + k - 1) * Wp, (long long)Ho * Wo)) {
    const unsigned x_len = (unsigned)(2 * ((long long)(B - 1) * x_ws + (long long)(H + k - 1) * Wp * C));
    const unsigned o_len = (unsigned)(2 * ((long long)(B - 1) * o_ws + (long long)Ho * Wo * C));
    const int R = dw_f16v_rows(k, s);
    // one channel pair a thread (5 x 5: 119 VGPRs with 6-row bands, 4 waves per SIMD; two pairs held 193 and ran 9 %
    // slower)
    if (dw_grid(Wo, dw_f16v_np(k, s), C / 2, (Ho + R - 1) / R, B, &nb, &total, &g)) return -1;
    dispatch_ks<h16>(k, s, [&]<int K, int S>() {
      constexpr int NP = dw_f16v_np(K, S), RR = dw_f16v_rows(K, S);
      hipLaunchKernelGGL((k_dw_f16v<K, S, 1, NP, RR, 1>), dim3(nb), dim3(256), 0, st, (const h16 *)xp, x_ws, x_len, Wp, C,
                         pt, pl, (const h16 *)w, (const h16 *)b, act, (h16 *)out, o_ws, o_len, Ho, Wo, total, g);
    });
    BNH_HIP(hipGetLastError());
    if (chsum) {
      BNH_REQ(B == 1 || cs_ws >= C);
      if (chsum_launch<h16, 1>((const h16 *)out, o_ws, C, Ho, Wo, chsum, cs_ws, B, st)) return -1;
    }
    return 0;
  }
  const bool pair = dw_pairs(xp, x_ws, w, b, out, o_ws, C, B);
  if (dw_grid(nit, dw_ni(k), pair ? C / 2 : C, Ho, B, &nb, &total, &g)) return -1;
  dispatch_ks<h16>(k, s, [&]<int K, int S>() {
    if (pair)
      hipLaunchKernelGGL((k_dw_f16p<K, S, 1>), dim3(nb), dim3(256), 0, st, (const h16 *)xp, x_ws, Wp, C, pt, pl,
                         (const h16 *)w, (const h16 *)b, act, (h16 *)out, o_ws, Ho, Wo, nit, total, g);
    else
      hipLaunchKernelGGL((k_dw_f16<K, S, 1>), dim3(nb), dim3(256), 0, st, (const h16 *)xp, x_ws, Wp, C, pt, pl,
                         (const h16 *)w, (const h16 *)b, act, (h16 *)out, o_ws, Ho, Wo, nit, total, g);
  });
  BNH_HIP(hipGetLastError());
  if (chsum) {
    BNH_REQ(B == 1 || cs_ws >= C);
    if (chsum_launch<h16, 1>((const h16 *)out, o_ws, C, Ho, Wo, chsum, cs_ws, B, st)) return -1;
  }
  return 0;
}

int bnh_dw3_f16(const uint16_t *xp, long long x_ws, int H, int W, int C, int s, int pt, int pl, const uint16_t *w,
                const uint16_t *b, uint16_t *out, long long o_ws, int Ho, int Wo, float *chsum, long long cs_ws, int B,
                void *stream) {
  BNH_REQ(xp && w && b && out && pt >= 0 && pt <= 1 && pl >= 0 && pl <= 1);
  if (dw_check(H, W, C, 3, s, pt, pl, Ho, Wo, B, x_ws, o_ws, 1)) return -1;
  const int nit = items_per_row(Wo, 2);
  unsigned nb;
  long long total;
  DwGrid g;
  hipStream_t st = bnh_stream(stream);
  if (dw_quads(xp, x_ws, w, b, out, o_ws, C, B, (long long)(H + 2) * (W + 2), (long long)Ho * Wo)) {
    const unsigned x_len = (unsigned)(2 * ((long long)(B - 1) * x_ws + (long long)(H + 2) * (W + 2) * C));
    const unsigned o_len = (unsigned)(2 * ((long long)(B - 1) * o_ws + (long long)Ho * Wo * C));
    const int R = dw_f16v_rows(3, s);
    if (dw_grid(Wo, dw3_f16v_np(s), C / 4, (Ho + R - 1) / R, B, &nb, &total, &g)) return -1;
    auto launch = [&]<int S>() {
      constexpr int NP = dw3_f16v_np(S), RR = dw_f16v_rows(3, S);
      hipLaunchKernelGGL((k_dw_f16v<3, S, 2, NP, RR, 2>), dim3(nb), dim3(256), 0, st, (const h16 *)xp, x_ws, x_len, W + 2, C,
                         pt, pl, (const h16 *)w, (const h16 *)b, 1, (h16 *)out, o_ws, o_len, Ho, Wo, total, g);
    };
    if (s == 1) launch.template operator()<1>();
    else launch.template operator()<2>();
    BNH_HIP(hipGetLastError());
    if (chsum) {
      BNH_REQ(B == 1 || cs_ws >= C);
      if (chsum_launch<h16, 3>((const h16 *)out, o_ws, C, Ho, Wo, chsum, cs_ws, B, st)) return -1;
    }
    return 0;
  }
  const bool pair = dw_pairs(xp, x_ws, w, b, out, o_ws, C, B);
  if (dw_grid(nit, dw_ni(3), pair ? C / 2 : C, Ho, B, &nb, &total, &g)) return -1;
#define DW3H(KERN, S_)                                                                                                 \
  hipLaunchKernelGGL((KERN<3, S_, 2>), dim3(nb), dim3(256), 0, st, (const h16 *)xp, x_ws, W + 2, C, pt, pl,           \
                     (const h16 *)w, (const h16 *)b, 1, (h16 *)out, o_ws, Ho, Wo, nit, total, g)
  if (pair) { if (s == 1) DW3H(k_dw_f16p, 1); else DW3H(k_dw_f16p, 2); }
  else { if (s == 1) DW3H(k_dw_f16, 1); else DW3H(k_dw_f16, 2); }
#undef DW3H
  BNH_HIP(hipGetLastError());
  if (chsum) {
    BNH_REQ(B == 1 || cs_ws >= C);
    if (chsum_launch<h16, 3>((const h16 *)out, o_ws, C, Ho, Wo, chsum, cs_ws, B, st)) return -1;
  }
  return 0;
}

}  // extern "C"

// BNH_DW_S8=strip runs stride-1 3x3 / 5x5 int8 depthwise convs on the strip kernel (k_dw_s8) instead of the
// row-streamed one (k_dw_s8_t), for comparison; results are the same bytes
static bool dw_s8_tiled() {
  static const bool tiled = [] {
    const char *e = getenv("BNH_DW_S8");
    return !(e && strcmp(e, "strip") == 0);
  }();
  return tiled;
}

extern "C" {
int bnh_dw_s8(const int8_t *x, long long x_ws, int H, int W, int C, int k, int s, int pt, int pl, const int8_t *w,
              const int32_t *bias, const int32_t *mult, const int32_t *shift, int zx, int zy, int lo, int hi,
              const int8_t *lut, int8_t *out, long long o_ws, int Ho, int Wo, int B, void *stream) {
  BNH_REQ(x && w && bias && mult && shift && out && H > 0 && W > 0 && Ho > 0 && Wo > 0 && B > 0);
  BNH_REQ(C > 0 && C % 4 == 0 && (k == 1 || k == 3 || k == 5 || k == 7) && (s == 1 || s == 2));
  BNH_REQ(pt >= 0 && pl >= 0 && pt < k && pl < k && lo >= -128 && hi <= 127 && lo <= hi);
  BNH_REQ(zx >= -128 && zx <= 127);
  BNH_REQ(((uintptr_t)x & 3) == 0 && ((uintptr_t)w & 3) == 0 && ((uintptr_t)out & 3) == 0);
  BNH_REQ(B == 1 || (x_ws % 4 == 0 && o_ws % 4 == 0 && x_ws >= (long long)H * W * C && o_ws >= (long long)Ho * Wo * C));
  // 32-bit buffer offsets: the batch's input and output each under 2 GiB
  const long long x_len = (long long)(B - 1) * x_ws + (long long)H * W * C;
  const long long o_len = (long long)(B - 1) * o_ws + (long long)Ho * Wo * C;
  BNH_REQ(x_len < (1LL << 31) && o_len < (1LL << 31) && (long long)k * k * C < (1LL << 31));
  hipStream_t st = bnh_stream(stream);
  // stride 1 with 3 x 3 or 5 x 5 taps: the LDS-tiled kernel
  if (s == 1 && (k == 3 || k == 5) && dw_s8_tiled()) {
    // 32 channels x 64 columns a block (64 or 128 channels with 32 or 16 columns measured the same or slower)
    auto launch = [&]<int K, int CT>() {
      constexpr int TW = 2048 / CT;
      const int ncg = (int)bnh_ceil_div(C, CT), ntx = (int)bnh_ceil_div(Wo, TW);
      const int nseg = (int)bnh_ceil_div(Ho, kDwtSeg);
      const long long nblk = (long long)ncg * ntx * nseg * B;
      if (nblk >= (1LL << 31)) return;
      if (lut)
        hipLaunchKernelGGL((k_dw_s8_t<K, CT, TW, true>), dim3((unsigned)nblk), dim3(256), 0, st, x, x_ws,
                           (unsigned)x_len, H, W, C, pt, pl, w, bias, mult, shift, zx, zy, lo, hi, lut, out, o_ws,
                           (unsigned)o_len, Ho, Wo, ncg, ntx, nseg);
      else
        hipLaunchKernelGGL((k_dw_s8_t<K, CT, TW, false>), dim3((unsigned)nblk), dim3(256), 0, st, x, x_ws,
                           (unsigned)x_len, H, W, C, pt, pl, w, bias, mult, shift, zx, zy, lo, hi, lut, out, o_ws,
                           (unsigned)o_len, Ho, Wo, ncg, ntx, nseg);
    };
    if (k == 3) launch.template operator()<3, 32>();
    else launch.template operator()<5, 32>();
    BNH_HIP(hipGetLastError());
    return 0;
  }
  unsigned nb;
  long long total;
  DwGrid g;
  if (dw_grid(Wo, dw_s8_np(s), C / 4, Ho, B, &nb, &total, &g)) return -1;
  dispatch_ks<int8_t>(k, s, [&]<int K, int S>() {
    if (lut)
      hipLaunchKernelGGL((k_dw_s8<K, S, true>), dim3(nb), dim3(256), 0, st, x, x_ws, (unsigned)x_len, H, W, C, pt, pl, w,
                         bias, mult, shift, zx, zy, lo, hi, lut, out, o_ws, (unsigned)o_len, Ho, Wo, total, g);
    else
      hipLaunchKernelGGL((k_dw_s8<K, S, false>), dim3(nb), dim3(256), 0, st, x, x_ws, (unsigned)x_len, H, W, C, pt, pl,
                         w, bias, mult, shift, zx, zy, lo, hi, lut, out, o_ws, (unsigned)o_len, Ho, Wo, total, g);
  });
  BNH_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
