/* CPU oracle (test infrastructure only): libbnneon's int8 Winograd F(2x2,3x3) (src/wino.c:26-227, the WINO_S8 op of
 * src/rt_ops_dot.c:130-170) for one window. See oracle.h. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static const int AT[2][4] = {{1, 1, 1, 0}, {0, 1, -1, -1}};

/* wino_pack (src/wino.c:26-88): U int8 [16][K][C] (position-major), sw [K], zw [4][K] */
void orc_wino8_pack(const float *w, int K, int C, int8_t *U8, float *sw, float *zw) {
  float *U = (float *)malloc(sizeof(float) * 16 * (size_t)K * C);
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
  int32_t *wsum = (int32_t *)calloc(16 * (size_t)K, sizeof(int32_t));
  for (int k = 0; k < K; k++) {
    float mx = 0;
    for (int xi = 0; xi < 16; xi++)
      for (int c = 0; c < C; c++) mx = fmaxf(mx, fabsf(U[((size_t)xi * K + k) * C + c]));
    const float s = mx > 0 ? mx / 127.f : 1.f;
    sw[k] = s;
    for (int xi = 0; xi < 16; xi++) {
      int32_t sum = 0;
      for (int c = 0; c < C; c++) {
        int v = (int)nearbyintf(U[((size_t)xi * K + k) * C + c] / s);
        v = v > 127 ? 127 : (v < -127 ? -127 : v);
        sum += v;
        U8[((size_t)xi * K + k) * C + c] = (int8_t)v;
      }
      wsum[xi * K + k] = sum;
    }
    for (int r = 0; r < 2; r++)
      for (int cc = 0; cc < 2; cc++) {
        long z = 0;
        for (int i = 0; i < 4; i++)
          for (int j = 0; j < 4; j++) z += (long)AT[r][i] * AT[cc][j] * wsum[(i * 4 + j) * K + k];
        zw[(r * 2 + cc) * K + k] = s * (float)z;
      }
  }
  free(wsum);
  free(U);
}

/* wino_f23_tiles (src/wino.c:135-227) over every tile of one window: x f32 [H][W][C] (zero padding: one pixel top /
 * left, the rest of the last tile bottom / right, as wino_f23_pad), out fp16 [H][W][K] */
void orc_wino8(const float *x, int H, int W, int C, int K, const int8_t *U8, const float *sw, const float *zw,
               const float *bias, uint16_t *out) {
  const int th = (H + 1) / 2, tw = (W + 1) / 2;
  float *V = (float *)malloc(sizeof(float) * 16 * (size_t)C);
  int8_t *q = (int8_t *)malloc(16 * (size_t)C);
  for (int ti = 0; ti < th; ti++)
    for (int tj = 0; tj < tw; tj++) {
      /* d[r][cc] = xp[2 ti + r][2 tj + cc], xp = x shifted by one pixel, zero outside */
      float mn = 0.f, mx = 0.f;
      for (int c = 0; c < C; c++) {
        float d[4][4], tm[4][4];
        for (int r = 0; r < 4; r++)
          for (int cc = 0; cc < 4; cc++) {
            const int y = 2 * ti + r - 1, xx = 2 * tj + cc - 1;
            d[r][cc] = (y >= 0 && y < H && xx >= 0 && xx < W) ? x[((size_t)y * W + xx) * C + c] : 0.f;
          }
        for (int cc = 0; cc < 4; cc++) {
          tm[0][cc] = d[0][cc] - d[2][cc]; tm[1][cc] = d[1][cc] + d[2][cc];
          tm[2][cc] = d[2][cc] - d[1][cc]; tm[3][cc] = d[1][cc] - d[3][cc];
        }
        for (int r = 0; r < 4; r++) {
          const float v0 = tm[r][0] - tm[r][2], v1 = tm[r][1] + tm[r][2];
          const float v2 = tm[r][2] - tm[r][1], v3 = tm[r][1] - tm[r][3];
          V[(r * 4 + 0) * C + c] = v0; V[(r * 4 + 1) * C + c] = v1;
          V[(r * 4 + 2) * C + c] = v2; V[(r * 4 + 3) * C + c] = v3;
          mn = orc_fmin(mn, orc_fmin(orc_fmin(v0, v1), orc_fmin(v2, v3)));
          mx = orc_fmax(mx, orc_fmax(orc_fmax(v0, v1), orc_fmax(v2, v3)));
        }
      }
      float s = (mx - mn) > 0 ? (mx - mn) / 255.f : 1.f;
      if (s < 1e-30f) s = 1e-30f;
      const float inv = 1.f / s, zp = nearbyintf(mn * inv) + 128.f;
      const int32_t zofs = (int32_t)((uint32_t)0x4B400000u + (uint32_t)orc_cvtz_s32(zp));
      for (int i = 0; i < 16 * C; i++) {
        const float m = fmaf(V[i], inv, 12582912.0f);
        uint32_t b;
        memcpy(&b, &m, 4);
        int32_t v = (int32_t)(b - (uint32_t)zofs);
        q[i] = (int8_t)(v < -128 ? -128 : v > 127 ? 127 : v);
      }
      const float sa = s, zs = s * zp;
      for (int k = 0; k < K; k++) {
        int32_t M[16];
        for (int xi = 0; xi < 16; xi++) {
          int32_t acc = 0;
          for (int c = 0; c < C; c++) acc += (int32_t)q[xi * C + c] * (int32_t)U8[((size_t)xi * K + k) * C + c];
          M[xi] = acc;
        }
        uint32_t s0[4], s1[4];
        for (int cc = 0; cc < 4; cc++) {
          s0[cc] = ((uint32_t)M[cc] + (uint32_t)M[4 + cc]) + (uint32_t)M[8 + cc];
          s1[cc] = ((uint32_t)M[4 + cc] - (uint32_t)M[8 + cc]) - (uint32_t)M[12 + cc];
        }
        const uint32_t Y[4] = {(s0[0] + s0[1]) + s0[2], (s0[1] - s0[2]) - s0[3], (s1[0] + s1[1]) + s1[2],
                               (s1[1] - s1[2]) - s1[3]};
        for (int o = 0; o < 4; o++) {
          const int oy = 2 * ti + o / 2, ox = 2 * tj + o % 2;
          if (oy >= H || ox >= W) continue;
          const float inner = fmaf((float)(int32_t)Y[o] * sw[k], sa, bias[k]);
          const float v = fmaf(zw[o * K + k], zs, inner);
          out[((size_t)oy * W + ox) * K + k] = orc_silu_lut_h(orc_f2h(v));
        }
      }
    }
  free(V);
  free(q);
}
