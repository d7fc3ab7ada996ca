/* The dotprod + fp16 family's kernels (src/rt_ops_dot.c) that the other files of the oracle do not cover. */
#include <math.h>
#include <string.h>

#include "oracle.h"

/* STEM3 (stem_conv_f32_h, src/kern_f16.c:15-71): img f32 [H][W][3], w OHWI [24][3][3][3], b [24] -> out fp16 bits,
 * zero-haloed [(H+1)/2 + 2][(W+1)/2 + 2][24] (the halo left as the caller zeroed it). Per output: acc = b[co], one
 * fmaf per tap (ky, kx, ci) in that order, taps past the bottom / right edge skipped (both paths of the reference
 * compute this chain), then FCVT to fp16 and the table SiLU. */
void orc_stem3_f32h(const float *img, int H, int W, const float *w, const float *b, uint16_t *out) {
  const int Ho = (H + 1) / 2, Wo = (W + 1) / 2;
  for (int oy = 0; oy < Ho; oy++)
    for (int ox = 0; ox < Wo; ox++)
      for (int co = 0; co < 24; co++) {
        float acc = b[co];
        for (int ky = 0; ky < 3; ky++) {
          const int iy = 2 * oy + ky;
          if (iy >= H) continue;
          for (int kx = 0; kx < 3; kx++) {
            const int ix = 2 * ox + kx;
            if (ix >= W) continue;
            for (int ci = 0; ci < 3; ci++)
              acc = fmaf(w[co * 27 + (ky * 3 + kx) * 3 + ci], img[((size_t)iy * W + ix) * 3 + ci], acc);
          }
        }
        out[((size_t)(oy + 1) * (Wo + 2) + ox + 1) * 24 + co] = orc_silu_lut_h(orc_f2h(acc));
      }
}
