// Registry kernels with fp16 arithmetic (variant 1, the reference's rt_ops_f16.c family) on the GPU.
#include "rt.h"

const rt_kernel *rt_k_f16(int base) {
  switch (base) {
    default: return nullptr;
  }
}
