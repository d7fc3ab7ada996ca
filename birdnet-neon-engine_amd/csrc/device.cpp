// Device plumbing of the kernel-level C ABI: errors, memory, streams, events, and the numerics probe.
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

extern "C" {

const char *bnh_last_error(void) { return g_err; }

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
