// The kernel registry: which op files serve each (opcode, variant). Variant 0 is the reference's fp32 / int8
// (no dotprod) family, variant 1 its fp16 family, variant 2 its dotprod + fp16 family (src/rt_pkg.c:320-331). An
// (opcode, variant) pair has one kernel.
#include "rt.h"

const rt_kernel *rt_k_s8n(int base);   // ops_s8n.cpp
const rt_kernel *rt_k_f32(int base);   // ops_f32.cpp
const rt_kernel *rt_k_f16(int base);   // ops_f16.cpp
const rt_kernel *rt_k_dot(int base);   // ops_dot.cpp

const rt_kernel *rt_k_var0(int base) {
  const rt_kernel *k = rt_k_s8n(base);
  return k ? k : rt_k_f32(base);
}
const rt_kernel *rt_k_var1(int base) { return rt_k_f16(base); }
const rt_kernel *rt_k_var2(int base) { return rt_k_dot(base); }
