// Registry kernels with fp32 arithmetic (variant 0 of the reference's rt_ops_f32.c family) on the GPU.
#include "rt.h"

const rt_kernel *rt_k_f32(int base) {
  switch (base) {
    default: return nullptr;
  }
}
