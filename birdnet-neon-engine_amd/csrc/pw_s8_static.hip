// bnh_pw_s8_static: the PW_S8 run of bnh_pw_s8 without a caller-provided workspace and without any allocation, for
// callers that cannot allocate device memory (code under HIP graph capture, serving loops that forbid hipMalloc).
//
// The quantized rows, row scales and zero points that bnh_pw_s8 takes as workspace arguments live here in one
// file-scope device array of BNH_PW_S8_STATIC_BYTES. Host code never passes the array's name to a kernel (in host
// code it is a stand-in, not a device address): its device address is looked up once per device with
// hipGetSymbolAddress on the first call made with that device current, and kept per device.
//
// Every call on a device shares that device's array and leaves its contents behind; nothing in it needs to start at
// zero (the quantize kernel writes every row, scale and zero point the GEMM reads, and the GEMM's row tail repeats
// the last written row). Calls that overlap on one device race on the array.
#include <mutex>

#include "bnh_internal.h"

#define BNH_PW_S8_STATIC_BYTES (64u << 20)
#define BNH_MAX_DEVICES 64

static __device__ __align__(256) unsigned char scratch[BNH_PW_S8_STATIC_BYTES];

static void *g_scratch[BNH_MAX_DEVICES];  // per device: the array's device address, once looked up
static std::mutex g_scratch_mu;

// the current device's address of `scratch` (looked up on the first call per device), or NULL with the error set
static unsigned char *scratch_ptr(void) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) { bnh_fail("bnh_pw_s8_static: hipGetDevice failed: %s", hipGetErrorString(e)); return nullptr; }
  if (dev < 0 || dev >= BNH_MAX_DEVICES) {
    bnh_fail("bnh_pw_s8_static: device %d: this library keeps the scratch address of devices 0..%d", dev,
             BNH_MAX_DEVICES - 1);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      bnh_fail("bnh_pw_s8_static: hipGetSymbolAddress of the scratch array failed on device %d: %s", dev,
               hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[dev] = p;
  }
  return (unsigned char *)g_scratch[dev];
}

extern "C" int bnh_pw_s8_static(const float *in, long long in_ws, int lda, int M, const float *gate, long long gate_ws,
                                int B, const bnh_s8w *W, const bnh_epi32 *e, void *stream) {
  BNH_REQ(in && W && e && M > 0 && B > 0);
  // the scratch layout: q int8 [B][M][Kp] (window stride M Kp, a multiple of 16), then sa f32 [B][M] and za i32
  // [B][M], each starting 256-byte aligned
  const unsigned long long rows = (unsigned long long)M * (unsigned long long)B;
  const unsigned long long qb = (rows * (unsigned long long)W->Kp + 255) & ~255ull;
  const unsigned long long sb = (rows * 4 + 255) & ~255ull;
  const unsigned long long need = qb + 2 * sb;
  if (need > BNH_PW_S8_STATIC_BYTES)
    return bnh_fail("bnh_pw_s8_static: %d windows x %d rows x (Kp %d + 8) bytes of quantized rows need %llu bytes of "
                    "scratch, more than its %u; hint: split the batch, or call bnh_pw_s8 with a workspace", B, M, W->Kp,
                    need, BNH_PW_S8_STATIC_BYTES);
  unsigned char *base = scratch_ptr();
  if (!base) return -1;
  int8_t *q = (int8_t *)base;
  float *sa = (float *)(base + qb);
  int32_t *za = (int32_t *)(base + qb + sb);
  const long long mk = (long long)M * W->Kp;
  return bnh_pw_s8(in, in_ws, lda, M, gate, gate_ws, q, mk, sa, M, za, M, B, W, e, stream);
}
