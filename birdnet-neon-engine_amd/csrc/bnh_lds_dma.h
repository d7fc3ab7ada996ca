// Direct global -> LDS loads (global_load_lds_dwordx4) and the waits that go with them, shared by the LDS-ring GEMMs.
//
// A wave's instruction copies 16 bytes per lane from the lane's own global address into 1 KB of LDS starting at the
// (wave-uniform) LDS address in M0, lane l at byte 16 l. The loads are issued from inline assembly and awaited with
// explicit vmcnt waits: the compiler, seeing an LDS-writing load, would otherwise wait for every outstanding load
// (vmcnt(0)) before each LDS read and serialise the ring. The "memory" clobbers keep the compiler from moving LDS
// accesses across the waits and the barriers. Vector-memory operations of a wave retire in issue order, so
// vmcnt(n) means "all but the n most recently issued have completed".
#ifndef BNH_LDS_DMA_H
#define BNH_LDS_DMA_H
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __attribute__((address_space(3))) int8_t lds_i8;

__device__ __forceinline__ void rq_dma16(const int8_t *src, const lds_i8 *dst) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}
// the saddr form: a wave-uniform 64-bit base (SGPRs) plus a 32-bit per-lane byte offset, so a ring whose lane
// offsets do not change from step to step spends no vector instruction on addresses
__device__ __forceinline__ void rq_dma16s(const void *base, uint32_t off, const lds_i8 *dst) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0) : "memory", "m0");
}
// the same for a stream read once (nt: non-temporal, so that it does not push L2-resident operands such as weights out)
__device__ __forceinline__ void rq_dma16s_nt(const void *base, uint32_t off, const lds_i8 *dst) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base), "s"(m0) : "memory", "m0");
}
#define RQ_WAIT_VM(n) asm volatile("s_waitcnt vmcnt(" #n ")" ::: "memory")
#define RQ_BARRIER() asm volatile("s_barrier" ::: "memory")

#endif
