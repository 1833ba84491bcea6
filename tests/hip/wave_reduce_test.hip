// Test-only kernels exercising csrc/wave_reduce.h on one wave64 (in bounds:
// exactly 64 threads, 64x64 inputs) and csrc/fast_trig.h (n elements, bounds
// checked), and calibration kernels of known VALU work for the hardware
// counters.  Built into tests/hip/libwave_test.so.
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

// Calibration kernels of known VALU work, for reading the SQ counters
// (SQ_INSTS_VALU, SQ_ACTIVE_INST_VALU, SQ_INSTS_VALU_TRANS_F32) against a
// count that is known: each thread runs `iters` iterations of 8 independent
// chains, one v_fma_f32 per chain per iteration (k_calib_fma), or one
// v_exp_f32 and one v_mul_f32 (k_calib_exp); the loop counter is scalar.
// 256 threads per block, one output per thread (in bounds by construction).
__global__ __launch_bounds__(256) void k_calib_fma(float* out, int iters, float a) {
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = static_cast<float>(threadIdx.x) * 1e-3f + i;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = fmaf(x[i], a, 0.5f);
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += x[i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}
__global__ __launch_bounds__(256) void k_calib_exp(float* out, int iters, float a) {
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = static_cast<float>(threadIdx.x) * 1e-3f + 0.1f * i;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = __builtin_amdgcn_exp2f(x[i]) * a;
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += x[i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}
// The render kernels' instruction mix: per iteration one v_exp_f32 and one
// v_mul_f32 on chain 0 and one v_fma_f32 on each of chains 1-7, all
// independent of each other within the iteration (9 VALU instructions, one
// of them transcendental).  Against k_calib_fma's 8 per iteration, its time
// shows whether a transcendental among independent VALU work holds its SIMD
// for two issue slots or overlaps with the instructions around it.
__global__ __launch_bounds__(256) void k_calib_mix(float* out, int iters, float a) {
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = static_cast<float>(threadIdx.x) * 1e-3f + 0.1f * i;
  for (int it = 0; it < iters; ++it) {
    x[0] = __builtin_amdgcn_exp2f(x[0]) * a;
#pragma unroll
    for (int i = 1; i < 8; ++i) x[i] = fmaf(x[i], a, 0.5f);
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += x[i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}
}  // namespace

// out: blocks * 256 floats.
extern "C" int calib_valu_fma(float* out, int blocks, int iters, float a, void* stream) {
  hipLaunchKernelGGL(k_calib_fma, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     out, iters, a);
  return static_cast<int>(hipGetLastError());
}

extern "C" int calib_valu_mix(float* out, int blocks, int iters, float a, void* stream) {
  hipLaunchKernelGGL(k_calib_mix, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     out, iters, a);
  return static_cast<int>(hipGetLastError());
}

extern "C" int calib_valu_exp(float* out, int blocks, int iters, float a, void* stream) {
  hipLaunchKernelGGL(k_calib_exp, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     out, iters, a);
  return static_cast<int>(hipGetLastError());
}

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
