// Test-only kernels exercising csrc/wave_reduce.h on one wave64 (in bounds:
// exactly 64 threads, 64x64 inputs) and csrc/fast_trig.h (n elements, bounds
// checked).  Built into tests/hip/libwave_test.so.
#include <hip/hip_runtime.h>

#include "fast_trig.h"
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
__global__ void k_sincos(const float* x, float* s, float* c, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) hrf::sincos_big(x[i], s + i, c + i);
}
}  // namespace

extern "C" int trig_test_sincos(const float* x, float* s, float* c, int n) {
  hipLaunchKernelGGL(k_sincos, dim3((n + 255) / 256), dim3(256), 0, nullptr, x, s, c, n);
  return static_cast<int>(hipDeviceSynchronize());
}

extern "C" int wave_test_transpose(const float* in, float* out) {
  hipLaunchKernelGGL(k_transpose, dim3(1), dim3(64), 0, nullptr, in, out);
  return static_cast<int>(hipDeviceSynchronize());
}

extern "C" int wave_test_sum(const float* in, float* out) {
  hipLaunchKernelGGL(k_sum, dim3(1), dim3(64), 0, nullptr, in, out);
  return static_cast<int>(hipDeviceSynchronize());
}
