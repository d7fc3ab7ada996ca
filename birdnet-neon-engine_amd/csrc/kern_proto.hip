// The int8 prototype head of libbnneon (PROTO_S8: src/proto_s8n.c, src/rt_ops_s8n.c:212-253, src/pc_kern_f32.c:364-374)
// on gfx950: per-cell symmetric int8 quantization of the L2-normalised cells, the cells x prototypes int8 MFMA GEMM
// whose epilogue keeps only the column maxima over each window's cells, and the class logits. Bit-identical to the
// reference (exact int32 sums; the max is exact and order-free; every float op as the reference rounds it).
//
// Prototypes are repacked at load from [Np/4][Kp/16][4][16] into rows [Npt][Kp] (Npt = Np rounded up to 256, zero
// rows past Np). A block computes one window's cells (row tiles of 64, running max) against 256 prototypes; blockIdx.x
// runs over windows so that concurrently resident blocks share one prototype tile.
#include <string.h>

#include "bnh_internal.h"
#include "bnh_num.h"

typedef int v4i __attribute__((ext_vector_type(4)));

struct bnh_s8p {
  int Np, Kp, Npt;
  int8_t *w;  // [Npt][Kp]
  float *sw;  // [Npt]
};

// ------------------------------------------------------------------ cell quantization (pc_quant_cells_f32)
// One wave per cell. The reference's sum of squares is 8 fused chains (channel c feeds chain c % 8, in order of c):
// lanes 0..7 run them over a 512-float LDS chunk the whole wave stages, then combine as ((t0 + t1) + (t2 + t3)),
// t_j = chain_j + chain_{j+4}. max |x| (FMAX, NaN-propagating) is order-free: all lanes, then a wave reduction.
#define QC_CHUNK 512
__global__ __launch_bounds__(256) void k_quant_cells(const float *__restrict__ x, long long x_ws, int P, int C, int ld,
                                                     float eps, int8_t *__restrict__ qa, long long qa_ws, int Kp,
                                                     float *__restrict__ sx, long long sx_ws, long long cells) {
  __shared__ float stage[4][QC_CHUNK];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const long long cell = (long long)blockIdx.x * 4 + wv;
  const bool live = cell < cells;
  const int w = live ? (int)(cell / P) : 0, p = live ? (int)(cell % P) : 0;
  const float *r = x + w * x_ws + (long long)p * ld;
  float chain = 0.f, mx = 0.f;
  for (int c0 = 0; c0 < C; c0 += QC_CHUNK) {
    const int n = C - c0 < QC_CHUNK ? C - c0 : QC_CHUNK;
    if (live)
      for (int i = lane; i < n; i += 64) {
        const float v = r[c0 + i];
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
        int32_t v = bnh_cvta_s32(r[c + j] * inv);
        v = v < -32768 ? -32768 : v > 32767 ? 32767 : v;
        v = v < -128 ? -128 : v > 127 ? 127 : v;
        b = v < -127 ? -127 : v;
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
  const int8_t *bp = wt + (long long)(n0 + (lane & 15)) * Kp + kc;
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
      for (int j = 0; j < 4; j++) b[j] = *(const v4i *)(bp + (long long)16 * j * Kp + k);
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
      for (int j = 0; j < 4; j++) b[j] = in ? *(const v4i *)(bp + (long long)16 * j * Kp + kmain) : (v4i){0, 0, 0, 0};
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
  const int Npt = (int)bnh_round_up(Np, 256);
  int8_t *hw = (int8_t *)calloc((size_t)Npt * Kp, 1);
  float *hs = (float *)calloc(Npt, 4);
  bnh_s8p *W = (bnh_s8p *)calloc(1, sizeof *W);
  if (!hw || !hs || !W) {
    free(hw); free(hs); free(W);
    bnh_fail("bnh_s8p_new: out of host memory");
    return nullptr;
  }
  const int kb = Kp / 16;
  for (int n = 0; n < Np; n++)
    for (int k = 0; k < Kp; k++) hw[(size_t)n * Kp + k] = qw[((size_t)(n / 4) * kb + k / 16) * 64 + (n % 4) * 16 + k % 16];
  memcpy(hs, sw, sizeof(float) * Np);
  W->Np = Np; W->Kp = Kp; W->Npt = Npt;
  bool ok = (W->w = (int8_t *)bnh_malloc((size_t)Npt * Kp)) && (W->sw = (float *)bnh_malloc(4 * (size_t)Npt)) &&
            !bnh_memcpy_h2d(W->w, hw, (size_t)Npt * Kp) && !bnh_memcpy_h2d(W->sw, hs, 4 * (size_t)Npt);
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
  hipLaunchKernelGGL(k_quant_cells, dim3((unsigned)bnh_ceil_div(cells, 4)), dim3(256), 0, bnh_stream(stream), x, x_ws, P,
                     C, ld, eps, qa, qa_ws, Kp, sx, sx_ws, cells);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_proto_colmax(const int8_t *qa, long long qa_ws, const float *sx, long long sx_ws, int P, const bnh_s8p *W,
                     float *colmax, long long cm_ws, int B, void *stream) {
  BNH_REQ(qa && sx && W && colmax && P > 0 && B > 0);
  BNH_REQ(((uintptr_t)qa & 15) == 0 && qa_ws % 16 == 0);
  BNH_REQ(B == 1 || (qa_ws >= (long long)P * W->Kp && cm_ws >= W->Np && sx_ws >= P));
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
