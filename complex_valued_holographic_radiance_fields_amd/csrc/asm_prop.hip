// asm_prop.hip — stage 4: band-limited angular-spectrum propagation around
// hipFFT, for gfx950.
//
// Transfer function.  The phase d*kz reaches ~1e5 rad, where one fp32 ulp is
// ~1e-2 rad, so kz must be reproduced bit-for-bit.  The recipe follows the
// reference host and kernel code (bandlimited_propagation_cuda.cu:60-72,
// 165-170): k = (float)(2*pi/(double)lambda); kz^2 = (float)((double)(k*k)
// - (2*pi*fx)^2 - (2*pi*fy)^2) with the products in double; kz =
// correctly-rounded sqrtf; phase = d*kz in float.  The frequencies are the
// float32 values of torch.fft.fftfreq: float(bin) * float(1/(M*pitch)),
// computed on the fly instead of read from two M x M grids.
//
// Shifts.  The reference multiplies fftshift(FFT) by the transfer function
// on the shifted grid and ifftshifts back (python_function.py:132-158).  The
// fused kernels work on the natural-order spectrum and map each natural
// index m to its shifted index (m + M/2) mod M for the frequency and the
// aperture, so no shift copies exist.
//
// Multi-plane fusion.  hologram[c] = sum_p iFFT(FFT(pad f[p,c]) T[p,c] A),
// and by linearity the sum over planes is taken in the spectral domain:
// P*C forward FFTs + C inverse FFTs per frame forward, C + P*C adjoint
// (the reference runs P*C forward and P*C inverse transforms per direction,
// plus an unused forward transform of the saved field in the backward).
#include <hipfft/hipfft.h>

#include <cmath>
#include <map>
#include <mutex>
#include <tuple>

#include "hrf_internal.h"

namespace hrf {
namespace {

constexpr double kTwoPi = 2.0 * 3.14159265358979323846;  // 2*M_PI in double

struct MacConsts {
  float k[kMaxChannels];
  float d[kMaxPlanes];
  float fxmax[kMaxPlanes * kMaxChannels];
  float fymax[kMaxPlanes * kMaxChannels];
};

// Transfer function value (cos, sin) or (0, 0), reference recipe.
__device__ __forceinline__ float2 transfer(float k, float fxv, float fyv, float fxmax,
                                          float fymax, float phase_d) {
  const bool within = (fabsf(fxv) < fxmax) && (fabsf(fyv) < fymax);
  const double a = kTwoPi * static_cast<double>(fxv);
  const double b = kTwoPi * static_cast<double>(fyv);
  const float kz2 = static_cast<float>((static_cast<double>(k * k) - a * a) - b * b);
  float2 tr = make_float2(0.0f, 0.0f);
  if (kz2 > 0.0f && within) {
    const float kz = sqrtf(kz2);
    const float ph = phase_d * kz;
    float sn, cs;
    sincosf(ph, &sn, &cs);
    tr = make_float2(cs, sn);
  }
  return tr;
}

__device__ __forceinline__ float2 cmul(float2 x, float2 y) {
  return make_float2(x.x * y.x - x.y * y.y, x.x * y.y + x.y * y.x);
}

// Drop-in kernel: grids and split re/im exactly as the reference binding.
__global__ void k_asm_grid(const float* __restrict__ re, const float* __restrict__ im,
                           const float* __restrict__ fxg, const float* __restrict__ fyg,
                           float* __restrict__ ore, float* __restrict__ oim, int nx, int ny,
                           float k, float fxmax, float fymax, float phase_d, float ap,
                           float offx, float offy) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  const int idy = blockIdx.y * blockDim.y + threadIdx.y;
  if (idx >= nx || idy >= ny) return;
  const int64_t index = static_cast<int64_t>(idy) * nx + idx;
  const float2 tr = transfer(k, fxg[index], fyg[index], fxmax, fymax, phase_d);
  float apv = 1.0f;
  if (ap > 0.0f) {
    const float x = static_cast<float>(idx) - offx;
    const float y = static_cast<float>(idy) - offy;
    apv = (x * x + y * y < ap * ap) ? 1.0f : 0.0f;
  }
  const float2 r = cmul(make_float2(re[index], im[index]), tr);
  ore[index] = r.x * apv;
  oim[index] = r.y * apv;
}

__device__ __forceinline__ void spectral_coords(int64_t elem, int M, float sfreq, float ap,
                                                float* fxv, float* fyv, float* apv) {
  const int mr = static_cast<int>(elem / M);
  const int mc = static_cast<int>(elem - static_cast<int64_t>(mr) * M);
  const int h = M / 2;
  int kr = mr + h;
  if (kr >= M) kr -= M;
  int kc = mc + h;
  if (kc >= M) kc -= M;
  *fxv = static_cast<float>(kr - h) * sfreq;  // rows carry FX (meshgrid 'ij')
  *fyv = static_cast<float>(kc - h) * sfreq;
  float a = 1.0f;
  if (ap > 0.0f) {
    const float off = static_cast<float>(M) / 2.0f - 0.5f;
    const float x = static_cast<float>(kc) - off;
    const float y = static_cast<float>(kr) - off;
    a = (x * x + y * y < ap * ap) ? 1.0f : 0.0f;
  }
  *apv = a;
}

// out[c] = sum_p spec[p,c] * T[p,c] * A   (natural-order spectra)
__global__ __launch_bounds__(256) void k_mac_fwd(const float2* __restrict__ spec, int P,
                                                 int C, int M, float sfreq, float ap,
                                                 MacConsts mc, float2* __restrict__ out) {
  const int64_t MM = static_cast<int64_t>(M) * M;
  const int64_t elem = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (elem >= MM) return;
  float fxv, fyv, apv;
  spectral_coords(elem, M, sfreq, ap, &fxv, &fyv, &apv);
  for (int c = 0; c < C; ++c) {
    float2 acc = make_float2(0.0f, 0.0f);
    if (apv != 0.0f) {
      for (int p = 0; p < P; ++p) {
        const float2 tr = transfer(mc.k[c], fxv, fyv, mc.fxmax[p * kMaxChannels + c],
                                   mc.fymax[p * kMaxChannels + c], mc.d[p]);
        const float2 x = spec[(static_cast<int64_t>(p) * C + c) * MM + elem];
        const float2 r = cmul(x, tr);
        acc.x += r.x;
        acc.y += r.y;
      }
    }
    out[static_cast<int64_t>(c) * MM + elem] = acc;
  }
}

// out[p,c] = spec[c] * conj(T[p,c]) * A  (phase -d*kz)
__global__ __launch_bounds__(256) void k_mac_adj(const float2* __restrict__ spec, int P,
                                                 int C, int M, float sfreq, float ap,
                                                 MacConsts mc, float2* __restrict__ out) {
  const int64_t MM = static_cast<int64_t>(M) * M;
  const int64_t elem = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (elem >= MM) return;
  float fxv, fyv, apv;
  spectral_coords(elem, M, sfreq, ap, &fxv, &fyv, &apv);
  for (int c = 0; c < C; ++c) {
    const float2 x = spec[static_cast<int64_t>(c) * MM + elem];
    for (int p = 0; p < P; ++p) {
      float2 r = make_float2(0.0f, 0.0f);
      if (apv != 0.0f) {
        const float2 tr = transfer(mc.k[c], fxv, fyv, mc.fxmax[p * kMaxChannels + c],
                                   mc.fymax[p * kMaxChannels + c], -mc.d[p]);
        r = cmul(x, tr);
      }
      out[(static_cast<int64_t>(p) * C + c) * MM + elem] = r;
    }
  }
}

// One distance of a multi-distance propagation: out[c] = spec[c] T[c] A
// with phase sign*d*kz (sign = +1 forward, -1 adjoint: conj(T)); with
// accumulate the product is added to out (the adjoint's sum over distances).
__global__ __launch_bounds__(256) void k_mac_dist(const float2* __restrict__ spec, int C, int M,
                                                  float sfreq, float ap, MacConsts mc,
                                                  float sign, int accumulate,
                                                  float2* __restrict__ out) {
  const int64_t MM = static_cast<int64_t>(M) * M;
  const int64_t elem = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (elem >= MM) return;
  float fxv, fyv, apv;
  spectral_coords(elem, M, sfreq, ap, &fxv, &fyv, &apv);
  for (int c = 0; c < C; ++c) {
    float2 r = make_float2(0.0f, 0.0f);
    if (apv != 0.0f) {
      const float2 tr = transfer(mc.k[c], fxv, fyv, mc.fxmax[c], mc.fymax[c], sign * mc.d[0]);
      r = cmul(spec[static_cast<int64_t>(c) * MM + elem], tr);
    }
    float2* o = out + static_cast<int64_t>(c) * MM + elem;
    if (accumulate) {
      const float2 prev = *o;
      r = make_float2(prev.x + r.x, prev.y + r.y);
    }
    *o = r;
  }
}

// Centred zero pad (batch,h,w) -> (batch,M,M); start = M/2 - n/2 as the
// reference's odak zero_pad (python_function.py:129).
__global__ void k_pad(const float2* __restrict__ in, int batch, int h, int w,
                      float2* __restrict__ out, int M) {
  const int64_t MM = static_cast<int64_t>(M) * M;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= MM * batch) return;
  const int64_t b = i / MM;
  const int64_t rem = i - b * MM;
  const int r = static_cast<int>(rem / M), c = static_cast<int>(rem - static_cast<int64_t>(r) * M);
  const int sr = r - (M / 2 - h / 2), sc = c - (M / 2 - w / 2);
  float2 v = make_float2(0.0f, 0.0f);
  if (sr >= 0 && sr < h && sc >= 0 && sc < w)
    v = in[(b * h + sr) * static_cast<int64_t>(w) + sc];
  out[i] = v;
}

// Centred crop (batch,M,M) -> (batch,h,w) times scale (crop_center,
// python_function.py:161,215; the 1/M^2 of torch.fft.ifft2).
__global__ void k_crop(const float2* __restrict__ in, int batch, int M, int h, int w,
                       float scale, float2* __restrict__ out) {
  const int64_t hw = static_cast<int64_t>(h) * w;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= hw * batch) return;
  const int64_t b = i / hw;
  const int64_t rem = i - b * hw;
  const int r = static_cast<int>(rem / w), c = static_cast<int>(rem - static_cast<int64_t>(r) * w);
  const int sr = r + (M / 2 - h / 2), sc = c + (M / 2 - w / 2);
  const float2 v = in[(b * M + sr) * static_cast<int64_t>(M) + sc];
  out[i] = make_float2(v.x * scale, v.y * scale);
}

MacConsts make_consts(int P, int C, int M, double pitch, const float* wl, const float* dist) {
  MacConsts mc{};
  for (int c = 0; c < C; ++c) {
    const AsmConsts a = asm_consts(wl[c], 0.0f, static_cast<float>(pitch), M, M);
    mc.k[c] = a.k;
  }
  for (int p = 0; p < P; ++p) {
    mc.d[p] = dist[p];
    for (int c = 0; c < C; ++c) {
      const AsmConsts a = asm_consts(wl[c], dist[p], static_cast<float>(pitch), M, M);
      mc.fxmax[p * kMaxChannels + c] = a.fx_max;
      mc.fymax[p * kMaxChannels + c] = a.fy_max;
    }
  }
  return mc;
}

float freq_step(int M, double pitch) {
  return static_cast<float>(1.0 / (static_cast<double>(M) * pitch));
}

// ------------------------------------------------------------- hipFFT --
struct PlanKey {
  int device, M, batch;
  bool operator<(const PlanKey& o) const {
    return std::tie(device, M, batch) < std::tie(o.device, o.M, o.batch);
  }
};
std::mutex g_plan_mu;
std::map<PlanKey, hipfftHandle>& plans() {
  static std::map<PlanKey, hipfftHandle> m;
  return m;
}

}  // namespace

AsmConsts asm_consts(float wavelength, float distance, float pixel_pitch, int nx, int ny) {
  AsmConsts a;
  a.k = static_cast<float>(kTwoPi / static_cast<double>(wavelength));
  const float x_size = pixel_pitch * static_cast<float>(nx);
  const float y_size = pixel_pitch * static_cast<float>(ny);
  const float tx = 2.0f * distance * (1.0f / x_size);
  const float ty = 2.0f * distance * (1.0f / y_size);
  a.fx_max = 1.0f / sqrtf(tx * tx + 1.0f) / wavelength;
  a.fy_max = 1.0f / sqrtf(ty * ty + 1.0f) / wavelength;
  a.dist = distance;
  a.pass = 1;
  return a;
}

int launch_asm_spectral_grid(const float* re, const float* im, const float* fxg,
                             const float* fyg, float* ore, float* oim, int nx, int ny,
                             float wavelength, float distance, float aperture, float pitch,
                             bool adjoint, hipStream_t s) {
  const AsmConsts a = asm_consts(wavelength, distance, pitch, nx, ny);
  const float offx = static_cast<float>(nx) / 2.0f - 0.5f;
  const float offy = static_cast<float>(ny) / 2.0f - 0.5f;
  dim3 block(16, 16);
  if (nx > 1024 && ny > 1024) block = dim3(32, 8);
  dim3 grid((nx + block.x - 1) / block.x, (ny + block.y - 1) / block.y);
  hipLaunchKernelGGL(k_asm_grid, grid, block, 0, s, re, im, fxg, fyg, ore, oim, nx, ny, a.k,
                     a.fx_max, a.fy_max, adjoint ? -distance : distance, aperture, offx, offy);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_asm_pad(const float2* in, int batch, int h, int w, float2* out, int M,
                   hipStream_t s) {
  const int64_t total = static_cast<int64_t>(M) * M * batch;
  hipLaunchKernelGGL(k_pad, dim3(blocks_for(total, 256)), dim3(256), 0, s, in, batch, h, w,
                     out, M);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_asm_crop(const float2* in, int batch, int M, int h, int w, float scale,
                    float2* out, hipStream_t s) {
  const int64_t total = static_cast<int64_t>(h) * w * batch;
  hipLaunchKernelGGL(k_crop, dim3(blocks_for(total, 256)), dim3(256), 0, s, in, batch, M, h,
                     w, scale, out);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_asm_mac_forward(const float2* spec, int P, int C, int M, double pitch,
                           const float* wavelengths, const float* distances, float aperture,
                           float2* out, hipStream_t s) {
  const MacConsts mc = make_consts(P, C, M, pitch, wavelengths, distances);
  const int64_t MM = static_cast<int64_t>(M) * M;
  hipLaunchKernelGGL(k_mac_fwd, dim3(blocks_for(MM, 256)), dim3(256), 0, s, spec, P, C, M,
                     freq_step(M, pitch), aperture, mc, out);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_asm_mac_adjoint(const float2* spec, int P, int C, int M, double pitch,
                           const float* wavelengths, const float* distances, float aperture,
                           float2* out, hipStream_t s) {
  const MacConsts mc = make_consts(P, C, M, pitch, wavelengths, distances);
  const int64_t MM = static_cast<int64_t>(M) * M;
  hipLaunchKernelGGL(k_mac_adj, dim3(blocks_for(MM, 256)), dim3(256), 0, s, spec, P, C, M,
                     freq_step(M, pitch), aperture, mc, out);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_asm_mac_distance(const float2* spec, int C, int M, double pitch,
                            const float* wavelengths, float distance, float aperture,
                            bool adjoint, bool accumulate, float2* out, hipStream_t s) {
  const MacConsts mc = make_consts(1, C, M, pitch, wavelengths, &distance);
  const int64_t MM = static_cast<int64_t>(M) * M;
  hipLaunchKernelGGL(k_mac_dist, dim3(blocks_for(MM, 256)), dim3(256), 0, s, spec, C, M,
                     freq_step(M, pitch), aperture, mc, adjoint ? -1.0f : 1.0f,
                     accumulate ? 1 : 0, out);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int fft_c2c(float2* buf, int M, int batch, bool inverse, hipStream_t s) {
  int dev = 0;
  HRF_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_plan_mu);
  const PlanKey key{dev, M, batch};
  auto it = plans().find(key);
  hipfftHandle plan;
  if (it == plans().end()) {
    int n[2] = {M, M};
    hipfftResult r = hipfftPlanMany(&plan, 2, n, nullptr, 1, M * M, nullptr, 1, M * M,
                                    HIPFFT_C2C, batch);
    if (r != HIPFFT_SUCCESS) {
      set_error("hipfftPlanMany(M=%d, batch=%d) failed with code %d", M, batch,
                static_cast<int>(r));
      return HRF_ERR_HIP;
    }
    plans()[key] = plan;
  } else {
    plan = it->second;
  }
  hipfftResult r = hipfftSetStream(plan, s);
  if (r != HIPFFT_SUCCESS) {
    set_error("hipfftSetStream failed with code %d", static_cast<int>(r));
    return HRF_ERR_HIP;
  }
  r = hipfftExecC2C(plan, reinterpret_cast<hipfftComplex*>(buf),
                    reinterpret_cast<hipfftComplex*>(buf),
                    inverse ? HIPFFT_BACKWARD : HIPFFT_FORWARD);
  if (r != HIPFFT_SUCCESS) {
    set_error("hipfftExecC2C(M=%d, batch=%d) failed with code %d", M, batch,
              static_cast<int>(r));
    return HRF_ERR_HIP;
  }
  return HRF_OK;
}

void fft_release_all() {
  std::lock_guard<std::mutex> lock(g_plan_mu);
  for (auto& kv : plans()) hipfftDestroy(kv.second);
  plans().clear();
}

}  // namespace hrf
