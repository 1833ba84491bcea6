// Test-only kernels exercising csrc/wave_reduce.h on one wave64 (in bounds:
// exactly 64 threads, 64x64 inputs).  Built into tests/hip/libwave_test.so.
#include <hip/hip_runtime.h>

#include "wave_reduce.h"

namespace {
__global__ __launch_bounds__(64) void k_transpose(const float* in, float* out) {
  float v[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) v[i] = in[threadIdx.x * 64 + i];
  out[threadIdx.x] = hrf::transpose_reduce64(v);
}
__global__ __launch_bounds__(64) void k_sum(const float* in, float* out) {
  out[threadIdx.x] = hrf::wave_sum_to_lane63(in[threadIdx.x]);
}
}  // namespace

extern "C" int wave_test_transpose(const float* in, float* out) {
  hipLaunchKernelGGL(k_transpose, dim3(1), dim3(64), 0, nullptr, in, out);
  return static_cast<int>(hipDeviceSynchronize());
}

extern "C" int wave_test_sum(const float* in, float* out) {
  hipLaunchKernelGGL(k_sum, dim3(1), dim3(64), 0, nullptr, in, out);
  return static_cast<int>(hipDeviceSynchronize());
}
