// Internal helpers shared by the libbnneon_hip sources (host side).
#ifndef BNH_INTERNAL_H
#define BNH_INTERNAL_H
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "bnneon_hip.h"

// thread-local message of the kernel-level API (bnh_last_error)
int bnh_fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void bnh_clear_error(void);

#define BNH_HIP(call)                                                                          \
  do {                                                                                         \
    hipError_t e_ = (call);                                                                    \
    if (e_ != hipSuccess) return bnh_fail("%s failed: %s", #call, hipGetErrorString(e_));      \
  } while (0)
#define BNH_REQ(cond)                                                                          \
  do {                                                                                         \
    if (!(cond)) return bnh_fail("%s: parameter check failed: %s", __func__, #cond);           \
  } while (0)

// the STEM kernel without the halo zeroing of bnh_stem_f32 (for outputs whose halo is known to be zero)
extern "C" int bnh_stem_f32_body(const float *img, long long i_ws, int H, int W, int k, int s, int Ho, int Wo, const float *w,
                      const float *bias, int Kp, int Np, int act, float *out, long long o_ws, int ldo, int opad, int B,
                      void *stream);

extern "C" int bnh_stem_f32to16_body(const float *img, long long i_ws, int H, int W, int k, int s, int Ho, int Wo,
                                     const float *w, const float *bias, int Kp, int N, int Np, int act, uint16_t *out,
                                     long long o_ws, int ldo, int opad, int B, void *stream);

// the int8 GEMM weights of PW_S8 / GEMV_S8 in HBM (kern_s8n.hip)
struct bnh_s8w {
  int N, K, Kp, Np, Nt;
  int8_t *w;        // [Nt][Kp]: channel rows, zero past Np
  float *sw, *b;    // [Nt]
  int32_t *colsum;  // [Nt]
};

// whether bnh_pwdw_f32 takes this expansion + depthwise pair (0) or not (-1, with the reason in bnh_last_error)
extern "C" int bnh_gemm_f16_mfma_body(const uint16_t *A, long long a_ws, int lda, int M, int B,
                                      const struct bnh_h16w *W, const bnh_epi16 *e, const uint16_t *gh,
                                      long long gh_ws, void *stream);

extern "C" int bnh_pwdw_f32_plan(int C, int Kp, int H, int W, int k, int s, int pt, int pl, int form, int Ho, int Wo);

static inline hipStream_t bnh_stream(void *s) { return (hipStream_t)s; }
static inline long long bnh_ceil_div(long long a, long long b) { return (a + b - 1) / b; }
static inline long long bnh_round_up(long long a, long long b) { return bnh_ceil_div(a, b) * b; }
#endif
