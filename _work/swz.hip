#include <hip/hip_runtime.h>
__global__ void k(float* o, const float* a) {
  float x = a[threadIdx.x], y = a[64 + threadIdx.x];
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  auto q = __builtin_amdgcn_permlane16_swap(r[0], r[1], false, false);
  o[threadIdx.x] = __uint_as_float(q[0]) + __uint_as_float(q[1]);
}
