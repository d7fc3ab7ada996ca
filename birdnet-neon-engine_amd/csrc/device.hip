// Device plumbing of the kernel-level C ABI: errors, memory, streams, events, and a streaming copy kernel (the
// bandwidth / counter calibration reference).
#include <string.h>

#include "bnh_internal.h"

static thread_local char g_err[512];

int bnh_fail(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return -1;
}
void bnh_clear_error(void) { g_err[0] = 0; }

// 16 bytes per thread per step, grid-stride: reads and writes each byte once
__global__ void k_copy16(const uint4 *__restrict__ src, uint4 *__restrict__ dst, long long n16) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (long long)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

extern "C" {

const char *bnh_last_error(void) { return g_err; }

int bnh_copy(void *dst, const void *src, size_t bytes, void *stream) {
  BNH_REQ(dst && src && bytes % 16 == 0 && ((uintptr_t)dst & 15) == 0 && ((uintptr_t)src & 15) == 0);
  const long long n16 = (long long)(bytes / 16);
  long long blocks = bnh_ceil_div(n16, 256);
  if (blocks > 256 * 64) blocks = 256 * 64;
  if (!n16) return 0;
  hipLaunchKernelGGL(k_copy16, dim3((unsigned)blocks), dim3(256), 0, bnh_stream(stream), (const uint4 *)src, (uint4 *)dst,
                     n16);
  BNH_HIP(hipGetLastError());
  return 0;
}

int bnh_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

void *bnh_malloc(size_t bytes) {
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
  if (e != hipSuccess) { bnh_fail("hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e)); return nullptr; }
  return p;
}
int bnh_free(void *p) {
  BNH_HIP(hipFree(p));
  return 0;
}
int bnh_memcpy_h2d(void *dst, const void *src, size_t bytes) {
  BNH_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return 0;
}
int bnh_memcpy_d2h(void *dst, const void *src, size_t bytes) {
  BNH_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return 0;
}
int bnh_memset(void *dst, int value, size_t bytes) {
  BNH_HIP(hipMemset(dst, value, bytes));
  return 0;
}
void *bnh_stream_new(void) {
  hipStream_t s = nullptr;
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) { bnh_fail("hipStreamCreate failed: %s", hipGetErrorString(e)); return nullptr; }
  return s;
}
int bnh_stream_free(void *s) {
  BNH_HIP(hipStreamDestroy(bnh_stream(s)));
  return 0;
}
int bnh_stream_sync(void *s) {
  BNH_HIP(hipStreamSynchronize(bnh_stream(s)));
  return 0;
}
void *bnh_event_new(void) {
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreate(&ev);
  if (e != hipSuccess) { bnh_fail("hipEventCreate failed: %s", hipGetErrorString(e)); return nullptr; }
  return ev;
}
int bnh_event_free(void *ev) {
  BNH_HIP(hipEventDestroy((hipEvent_t)ev));
  return 0;
}
int bnh_event_record(void *ev, void *s) {
  BNH_HIP(hipEventRecord((hipEvent_t)ev, bnh_stream(s)));
  return 0;
}
float bnh_event_ms(void *a, void *b) {
  float ms = -1.f;
  hipError_t e = hipEventElapsedTime(&ms, (hipEvent_t)a, (hipEvent_t)b);
  if (e != hipSuccess) { bnh_fail("hipEventElapsedTime failed: %s", hipGetErrorString(e)); return -1.f; }
  return ms;
}

}  // extern "C"
