// recon.hip — the loss side's hologram reconstruction around the
// propagation: the per-(frame, channel) hologram field from the phase map and
// the amplitude, the reconstructed intensity |u|^2, and the backward of both.
//
// Reference: propagator._reconstruct_impl (utils/propagator.py:548-636):
// for every frame f and channel c with laser power w = laser_powers[f][c],
// hologram = generate_complex_field(w * amplitude[c], phase[f] *
// phase_scale[c]) (= w a e^{i s phi}), zero pad, propagate to every depth,
// crop, then calculate_amplitude(.)**2.  Only pairs with w != 0 are formed
// (the reference's training uses laser_channel_power = eye(3): one channel
// per frame), as K fields in one array; the propagation between these
// kernels is the multi-distance band-limited ASM.
#include <cmath>

#include "hrf_internal.h"

namespace hrf {
namespace {

constexpr int kReconThreads = 256;
constexpr int kMaxReconPairs = 64;

struct ReconPairs {
  int frame[kMaxReconPairs];
  int channel[kMaxReconPairs];
  float power[kMaxReconPairs];
  float scale[kMaxReconPairs];  // phase_scale[channel]
  int count;
};

// fields[k][i] = power_k * amp[c_k][i] * e^{i scale_k * phase[f_k][i]}
__global__ __launch_bounds__(kReconThreads) void k_recon_fields(
    const float* __restrict__ amp, const float* __restrict__ phase, int64_t hw, ReconPairs pr,
    float2* __restrict__ fields) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kReconThreads + threadIdx.x;
  const int k = blockIdx.y;
  if (i >= hw) return;
  const float a = pr.power[k] * amp[static_cast<int64_t>(pr.channel[k]) * hw + i];
  const float th = phase[static_cast<int64_t>(pr.frame[k]) * hw + i] * pr.scale[k];
  float s, c;
  sincosf(th, &s, &c);
  fields[static_cast<int64_t>(k) * hw + i] = make_float2(a * c, a * s);
}

__global__ __launch_bounds__(kReconThreads) void k_recon_intensity(const float2* __restrict__ u,
                                                                   int64_t n,
                                                                   float* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kReconThreads + threadIdx.x;
  if (i >= n) return;
  const float2 v = u[i];
  out[i] = v.x * v.x + v.y * v.y;
}

// d|u|^2: grad_u = 2 g u (torch's convention for a real loss of complex u).
__global__ __launch_bounds__(kReconThreads) void k_recon_intensity_bwd(
    const float2* __restrict__ u, const float* __restrict__ g, int64_t n,
    float2* __restrict__ gu) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kReconThreads + threadIdx.x;
  if (i >= n) return;
  const float2 v = u[i];
  const float t = 2.0f * g[i];
  gu[i] = make_float2(t * v.x, t * v.y);
}

// z = w a e^{i s phi}: dL/da = w Re(gz e^{-i s phi}), dL/dphi = s Im(gz conj(z))
// summed over the pairs that use the channel / frame (each pixel loops over
// the pairs, so there are no atomics).
__global__ __launch_bounds__(kReconThreads) void k_recon_fields_bwd(
    const float* __restrict__ amp, const float* __restrict__ phase, int64_t hw, ReconPairs pr,
    const float2* __restrict__ gfields, int F, int C, float* __restrict__ g_amp,
    float* __restrict__ g_phase) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kReconThreads + threadIdx.x;
  if (i >= hw) return;
  for (int c = 0; c < C; ++c) g_amp[static_cast<int64_t>(c) * hw + i] = 0.0f;
  for (int f = 0; f < F; ++f) g_phase[static_cast<int64_t>(f) * hw + i] = 0.0f;
  for (int k = 0; k < pr.count; ++k) {
    const int64_t ic = static_cast<int64_t>(pr.channel[k]) * hw + i;
    const int64_t jf = static_cast<int64_t>(pr.frame[k]) * hw + i;
    const float th = phase[jf] * pr.scale[k];
    float s, c;
    sincosf(th, &s, &c);
    const float2 gz = gfields[static_cast<int64_t>(k) * hw + i];
    const float re = gz.x * c + gz.y * s;    // Re(gz e^{-i th})
    const float im = gz.y * c - gz.x * s;    // Im(gz e^{-i th})
    const float a = pr.power[k] * amp[ic];
    g_amp[ic] += pr.power[k] * re;
    g_phase[jf] += pr.scale[k] * a * im;     // Im(gz conj(z)) = a Im(gz e^{-i th})
  }
}

int pairs_of(const int32_t* frames, const int32_t* channels, const float* powers,
             const float* scales, int32_t K, int F, int C, ReconPairs* pr) {
  if (K < 1 || K > kMaxReconPairs || !frames || !channels || !powers || !scales) {
    set_error("reconstruction: 1..%d (frame, channel) pairs needed", kMaxReconPairs);
    return HRF_ERR_INVALID;
  }
  *pr = ReconPairs{};
  for (int k = 0; k < K; ++k) {
    if (frames[k] < 0 || frames[k] >= F || channels[k] < 0 || channels[k] >= C) {
      set_error("reconstruction: pair %d = (%d, %d) outside %d frames x %d channels", k,
                frames[k], channels[k], F, C);
      return HRF_ERR_INVALID;
    }
    pr->frame[k] = frames[k];
    pr->channel[k] = channels[k];
    pr->power[k] = powers[k];
    pr->scale[k] = scales[k];
  }
  pr->count = K;
  return HRF_OK;
}

}  // namespace
}  // namespace hrf

using namespace hrf;

extern "C" {

int hrf_recon_fields(const float* amplitude, const float* phase, int32_t F, int32_t C,
                     int64_t hw, const int32_t* frames, const int32_t* channels,
                     const float* powers, const float* scales, int32_t K, void* fields,
                     void* stream) {
  ReconPairs pr;
  HRF_TRY(pairs_of(frames, channels, powers, scales, K, F, C, &pr));
  if (hw <= 0 || !amplitude || !phase || !fields) {
    set_error("reconstruction fields: invalid size or null pointer");
    return HRF_ERR_INVALID;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  HRF_STAGE("recon_fields", s);
  hipLaunchKernelGGL(k_recon_fields, dim3(blocks_for(hw, kReconThreads), K),
                     dim3(kReconThreads), 0, s, amplitude, phase, hw, pr,
                     static_cast<float2*>(fields));
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int hrf_recon_intensity(const void* field, int64_t n, float* intensity, void* stream) {
  if (n < 0 || (n > 0 && (!field || !intensity))) {
    set_error("reconstruction intensity: invalid size or null pointer");
    return HRF_ERR_INVALID;
  }
  if (n == 0) return HRF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  HRF_STAGE("recon_intensity", s);
  hipLaunchKernelGGL(k_recon_intensity, dim3(blocks_for(n, kReconThreads)), dim3(kReconThreads),
                     0, s, static_cast<const float2*>(field), n, intensity);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int hrf_recon_intensity_backward(const void* field, const float* grad_intensity, int64_t n,
                                 void* grad_field, void* stream) {
  if (n < 0 || (n > 0 && (!field || !grad_intensity || !grad_field))) {
    set_error("reconstruction intensity backward: invalid size or null pointer");
    return HRF_ERR_INVALID;
  }
  if (n == 0) return HRF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  HRF_STAGE("recon_intensity", s);
  hipLaunchKernelGGL(k_recon_intensity_bwd, dim3(blocks_for(n, kReconThreads)),
                     dim3(kReconThreads), 0, s, static_cast<const float2*>(field),
                     grad_intensity, n, static_cast<float2*>(grad_field));
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int hrf_recon_fields_backward(const float* amplitude, const float* phase, int32_t F, int32_t C,
                              int64_t hw, const int32_t* frames, const int32_t* channels,
                              const float* powers, const float* scales, int32_t K,
                              const void* grad_fields, float* grad_amplitude,
                              float* grad_phase, void* stream) {
  ReconPairs pr;
  HRF_TRY(pairs_of(frames, channels, powers, scales, K, F, C, &pr));
  if (hw <= 0 || !amplitude || !phase || !grad_fields || !grad_amplitude || !grad_phase) {
    set_error("reconstruction fields backward: invalid size or null pointer");
    return HRF_ERR_INVALID;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  HRF_STAGE("recon_fields", s);
  hipLaunchKernelGGL(k_recon_fields_bwd, dim3(blocks_for(hw, kReconThreads)), dim3(kReconThreads),
                     0, s, amplitude, phase, hw, pr, static_cast<const float2*>(grad_fields), F,
                     C, grad_amplitude, grad_phase);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

}  // extern "C"
