// Kernels of the dotprod + fp16 family's ops (src/rt_ops_dot.c) that have no kernel file of their own here.
//
// STEM3 (src/rt_ops_dot.c:46-61; stem_conv_f32_h, src/kern_f16.c:15-71): 3 x 3 stride-2 convolution of a
// 3-channel fp32 image [H][W][3] into 24 channels. For an even H and W the TF-same pads are bottom / right only:
// taps past the image are skipped. Per output one fp32 FMA chain from b[co] over the taps (ky, kx, ci) in order,
// rounded to fp16 (nearest even), then the table SiLU, into the zero-haloed fp16 [Ho+2][Wo+2][24]. A thread owns 8
// channels of one output pixel (one 16-byte store).
#include "bnh_internal.h"
#include "bnh_num.h"
#include "bnh_f16.h"

__global__ __launch_bounds__(256) void k_stem3(const float *__restrict__ img, long long i_ws, int H, int W,
                                               const float *__restrict__ w, const float *__restrict__ b,
                                               uint16_t *__restrict__ out, long long o_ws, int Ho, int Wo,
                                               long long total) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int g = (int)(i % 3);
  long long r = i / 3;
  const int ox = (int)(r % Wo);
  r /= Wo;
  const int oy = (int)(r % Ho), win = (int)(r / Ho);
  const int c0 = 8 * g;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; j++) acc[j] = b[c0 + j];
  const float *im = img + win * i_ws;
#pragma unroll
  for (int ky = 0; ky < 3; ky++) {
    const int iy = 2 * oy + ky;
    if (iy >= H) continue;
#pragma unroll
    for (int kx = 0; kx < 3; kx++) {
      const int ix = 2 * ox + kx;
      if (ix >= W) continue;
      const float *p = im + ((long long)iy * W + ix) * 3;
#pragma unroll
      for (int ci = 0; ci < 3; ci++) {
        const float v = p[ci];
        const int t = (ky * 3 + kx) * 3 + ci;
#pragma unroll
        for (int j = 0; j < 8; j++) acc[j] = __builtin_fmaf(w[(c0 + j) * 27 + t], v, acc[j]);
      }
    }
  }
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
    o[j] = (uint32_t)hbits(silu_lut_h(f2h(acc[2 * j]))) | ((uint32_t)hbits(silu_lut_h(f2h(acc[2 * j + 1]))) << 16);
  *(uint4 *)(out + win * o_ws + ((long long)(oy + 1) * (Wo + 2) + ox + 1) * 24 + c0) = make_uint4(o[0], o[1], o[2], o[3]);
}

extern "C" int bnh_stem3_f16(const float *img, long long i_ws, int H, int W, const float *w, const float *b,
                             uint16_t *out, long long o_ws, int B, void *stream) {
  BNH_REQ(img && w && b && out && H > 0 && W > 0 && B > 0);
  const int Ho = (H + 1) / 2, Wo = (W + 1) / 2;
  BNH_REQ(((uintptr_t)out & 15) == 0 && (B == 1 || (i_ws >= (long long)H * W * 3 && o_ws % 8 == 0 &&
                                                    o_ws >= (long long)(Ho + 2) * (Wo + 2) * 24)));
  const long long total = (long long)B * Ho * Wo * 3;
  BNH_REQ(bnh_ceil_div(total, 256) < (1LL << 31));
  hipLaunchKernelGGL(k_stem3, dim3((unsigned)bnh_ceil_div(total, 256)), dim3(256), 0, bnh_stream(stream), img, i_ws,
                     H, W, w, b, out, o_ws, Ho, Wo, total);
  BNH_HIP(hipGetLastError());
  return 0;
}
