// Test-only kernels exercising csrc/wave_reduce.h on one wave64 (in bounds:
// exactly 64 threads, 64x64 or 64x12 inputs) and csrc/fast_trig.h (n elements, bounds
// checked), and calibration kernels of known VALU work for the hardware
// counters.  Built into tests/hip/libwave_test.so.
#include <hip/hip_runtime.h>

#include "fast_trig.h"
#include "render_member.h"
#include "wave_reduce.h"

namespace {
__global__ __launch_bounds__(64) void k_transpose(const float* in, float* out) {
  float v[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) v[i] = in[threadIdx.x * 64 + i];
  out[threadIdx.x] = hrf::transpose_reduce64(v);
}
// row_sum16 over 12 values per lane: lane L writes its 3 sums to
// out[L * 3 .. L * 3 + 3).
__global__ __launch_bounds__(64) void k_row_sum16(const float* in, float* out) {
  float v[12];
#pragma unroll
  for (int i = 0; i < 12; ++i) v[i] = in[threadIdx.x * 12 + i];
  float x[3];
  hrf::row_sum16<12>(v, x);
#pragma unroll
  for (int i = 0; i < 3; ++i) out[threadIdx.x * 3 + i] = x[i];
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
// As k_calib_fma, with the two factors in VGPRs: x = fma(u, v, x) compiles
// to the 4-byte VOP2 v_fmac_f32 (k_calib_fma's fma(x, a, 0.5) with a scalar
// operand and a constant is the 8-byte VOP3 v_fma_f32).
__global__ __launch_bounds__(256) void k_calib_fmac(float* out, int iters, float a) {
  float x[8];
  const float u = a * 1e-3f * static_cast<float>(threadIdx.x & 7);
  const float v = 1e-3f * static_cast<float>(threadIdx.x >> 3);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = static_cast<float>(threadIdx.x) * 1e-3f + i;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = fmaf(u, v, x[i]);
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
// The forward render's fast member loop (hrf::fwd_member, C = 3), as
// k_render_fwd runs it: 256 staged members per batch in LDS (3 quads each),
// walked 8 at a time with the per-group all-done vote, one pixel per lane.
// The members are synthetic and faint (alpha ~ 2^-20), so no lane ever
// terminates and every iteration runs the whole batch: the counted VALU
// instructions over the kernel's time give the issue rate this instruction
// mix reaches on its own (no staging, barriers or memory).
__global__ __launch_bounds__(256, 8) void k_calib_fwdloop(float* out, int iters) {
  __shared__ float4 s_rec[256 * 3];
  const int tid = threadIdx.x;
  {
    const float fi = static_cast<float>(tid);
    // (c0, c1, c2, c3), (c4, c5, re0, im0), (re1, im1, re2, im2): an
    // exponent near -20 over the tile
    s_rec[tid * 3] = make_float4(-20.0f + 0.001f * fi, 0.01f, -0.01f, -0.002f);
    s_rec[tid * 3 + 1] = make_float4(0.001f, -0.003f, 0.5f, 0.25f);
    s_rec[tid * 3 + 2] = make_float4(0.125f, -0.5f, 0.75f, 0.3f);
  }
  __syncthreads();
  const float pxf = static_cast<float>(tid & 15) - 7.5f, pyf = static_cast<float>(tid >> 4) - 7.5f;
  float T = 1.0f, acc[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int evaluated = 0;
  for (int it = 0; it < iters; ++it) {
    for (int j0 = 0; j0 < 256; j0 += 8) {
      if (__all(T < hrf::kTermT)) break;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int j = j0 + jj;
        hrf::fwd_member<3>(s_rec[j * 3], s_rec[j * 3 + 1], s_rec[j * 3 + 2], pxf, pyf, T, acc,
                           evaluated);
      }
    }
  }
  float sum = T + static_cast<float>(evaluated);
#pragma unroll
  for (int i = 0; i < 6; ++i) sum += acc[i];
  out[blockIdx.x * 256 + tid] = sum;
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

extern "C" int calib_valu_fwdloop(float* out, int blocks, int iters, float a, void* stream) {
  (void)a;
  hipLaunchKernelGGL(k_calib_fwdloop, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), out, iters);
  return static_cast<int>(hipGetLastError());
}

extern "C" int calib_valu_fmac(float* out, int blocks, int iters, float a, void* stream) {
  hipLaunchKernelGGL(k_calib_fmac, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
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

extern "C" int wave_test_row_sum16(const float* in, float* out) {
  hipLaunchKernelGGL(k_row_sum16, dim3(1), dim3(64), 0, nullptr, in, out);
  return static_cast<int>(hipDeviceSynchronize());
}

extern "C" int wave_test_sum(const float* in, float* out) {
  hipLaunchKernelGGL(k_sum, dim3(1), dim3(64), 0, nullptr, in, out);
  return static_cast<int>(hipDeviceSynchronize());
}
