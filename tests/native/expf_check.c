/* Compares bnh_expf (the device header, compiled for the host) with the C library's expf on floats
 * [lo, hi) of the 2^32 bit patterns, striding by `step`, over `threads` threads. Prints the mismatch count and the
 * first mismatches; exits 0 iff there are none. */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "bnh_expf.h"

typedef struct { uint64_t lo, hi, step; uint64_t bad; uint32_t first; } job;

static void *run(void *a) {
  job *j = a;
  j->bad = 0;
  for (uint64_t u = j->lo; u < j->hi; u += j->step) {
    uint32_t b = (uint32_t)u;
    float x, y0, y1;
    memcpy(&x, &b, 4);
    y0 = expf(x);
    y1 = bnh_expf(x);
    uint32_t p, q;
    memcpy(&p, &y0, 4);
    memcpy(&q, &y1, 4);
    if (p != q && !(y0 != y0 && y1 != y1)) {
      if (!j->bad) j->first = b;
      j->bad++;
    }
  }
  return NULL;
}

int main(int argc, char **argv) {
  uint64_t step = argc > 1 ? strtoull(argv[1], 0, 0) : 1;
  int nt = argc > 2 ? atoi(argv[2]) : 8;
  pthread_t th[64];
  job jb[64];
  const uint64_t total = 1ull << 32, chunk = total / nt;
  for (int i = 0; i < nt; i++) {
    jb[i].lo = i * chunk;
    jb[i].hi = i == nt - 1 ? total : (i + 1) * chunk;
    jb[i].lo += (step - jb[i].lo % step) % step;
    jb[i].step = step;
    pthread_create(&th[i], NULL, run, &jb[i]);
  }
  uint64_t bad = 0;
  for (int i = 0; i < nt; i++) {
    pthread_join(th[i], NULL);
    if (jb[i].bad) printf("first mismatch in part %d: 0x%08x\n", i, jb[i].first);
    bad += jb[i].bad;
  }
  printf("mismatches %llu\n", (unsigned long long)bad);
  return bad != 0;
}
