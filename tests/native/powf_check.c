/* Compares bnh_powf (the device header, compiled for the host) with the C library's powf, over `threads` threads:
 *   1. every `stride`-th float x in [2^-130, 2^8) (subnormals through the means GEM_A produces) with y = 1/p for p in
 *      {1, 1.5, 2, 2.5, 3, 3.5, 4, 5, 6, 8, 10}, y rounded to float as the reference's 1.0f / p is;
 *   2. `nrand` pseudo-random pairs (x, y) over every finite bit pattern of x and |y| <= 64;
 *   3. the special cases: zeros, infinities, NaNs, negative x with integer and non-integer y, 1 and -1.
 * Prints the mismatch count and the first mismatches; exits 0 iff there are none. */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "bnh_powf.h"

static const float kP[] = {1.f, 1.5f, 2.f, 2.5f, 3.f, 3.5f, 4.f, 5.f, 6.f, 8.f, 10.f};
#define NP (sizeof kP / sizeof kP[0])

typedef struct { uint32_t lo, hi, stride; uint64_t nrand, seed; uint64_t bad, n; float fx, fy; } job;

static int differ(float x, float y) {
  const float a = powf(x, y), b = bnh_powf(x, y);
  uint32_t p, q;
  memcpy(&p, &a, 4);
  memcpy(&q, &b, 4);
  return p != q && !(a != a && b != b);
}

static uint64_t next(uint64_t *s) {  /* splitmix64 */
  uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

static void note(job *j, float x, float y) {
  if (!j->bad) { j->fx = x; j->fy = y; }
  j->bad++;
}

static void *run(void *a) {
  job *j = a;
  for (uint32_t u = j->lo; u < j->hi; u += j->stride) {
    float x;
    memcpy(&x, &u, 4);
    for (unsigned i = 0; i < NP; i++) {
      const float y = 1.0f / kP[i];
      j->n++;
      if (differ(x, y)) note(j, x, y);
    }
  }
  uint64_t s = j->seed;
  for (uint64_t i = 0; i < j->nrand; i++) {
    const uint64_t v = next(&s);
    uint32_t ux = (uint32_t)v, uy = (uint32_t)(v >> 32);
    if ((ux & 0x7f800000u) == 0x7f800000u) ux &= 0xbfffffffu;  /* finite x */
    float x, y;
    memcpy(&x, &ux, 4);
    y = (float)((int32_t)uy) * 0x1p-25f;                       /* |y| <= 64 */
    if (uy & 1) y = truncf(y);                                  /* integer y half the time */
    j->n++;
    if (differ(x, y)) note(j, x, y);
  }
  return NULL;
}

int main(int argc, char **argv) {
  const uint64_t nrand = argc > 1 ? strtoull(argv[1], 0, 0) : 20000000;
  int nt = argc > 2 ? atoi(argv[2]) : 8;
  if (nt < 1) nt = 1;
  if (nt > 64) nt = 64;
  const uint32_t stride = argc > 3 ? (uint32_t)strtoul(argv[3], 0, 0) : 1;
  const uint32_t lo = 0x00400000u, hi = 0x43800000u;  /* 2^-130 .. 2^8 */
  pthread_t th[64];
  job jb[64];
  memset(jb, 0, sizeof jb);
  for (int i = 0; i < nt; i++) {
    jb[i].lo = lo + (uint32_t)((uint64_t)(hi - lo) * i / nt);
    jb[i].hi = lo + (uint32_t)((uint64_t)(hi - lo) * (i + 1) / nt);
    jb[i].stride = stride ? stride : 1;
    jb[i].nrand = nrand / nt;
    jb[i].seed = 0x5eed + i;
    pthread_create(&th[i], NULL, run, &jb[i]);
  }
  uint64_t bad = 0, n = 0;
  for (int i = 0; i < nt; i++) {
    pthread_join(th[i], NULL);
    if (jb[i].bad) printf("first mismatch in part %d: powf(%a, %a)\n", i, jb[i].fx, jb[i].fy);
    bad += jb[i].bad;
    n += jb[i].n;
  }
  static const float sx[] = {0.f, -0.f, 1.f, -1.f, 2.f, -2.f, 0.5f, -0.5f, INFINITY, -INFINITY, NAN, -NAN, 0x1p-149f,
                             -0x1p-149f, 0x1p127f, -3.f, 1e-30f};
  static const float sy[] = {0.f, -0.f, 1.f, -1.f, 2.f, -2.f, 3.f, -3.f, 0.5f, -0.5f, INFINITY, -INFINITY, NAN, 1.5f,
                             200.f, -200.f, 0x1p-149f, 1e30f};
  for (unsigned a = 0; a < sizeof sx / sizeof sx[0]; a++)
    for (unsigned b = 0; b < sizeof sy / sizeof sy[0]; b++) {
      n++;
      if (differ(sx[a], sy[b])) {
        if (bad < 8) printf("special mismatch: powf(%a, %a) = %a, restated %a\n", sx[a], sy[b], powf(sx[a], sy[b]),
                            bnh_powf(sx[a], sy[b]));
        bad++;
      }
    }
  printf("compared %llu, mismatches %llu\n", (unsigned long long)n, (unsigned long long)bad);
  return bad != 0;
}
