// fast_trig.h — sine and cosine of large float arguments for the transfer
// function of the propagation kernels.
//
// The phase d*kz is formed in float exactly as the reference forms it and
// reaches ~1e4-1e5 rad.  Its sine and cosine are taken here by reducing the
// float argument modulo 2*pi in double precision (x is exact as a double and
// x/(2*pi) keeps 53 bits, so the fractional revolution is accurate to ~1e-12)
// and evaluating the hardware sin/cos of that fraction in revolutions
// (v_sin_f32 / v_cos_f32 compute sin(2*pi*r)).  Absolute error is a few 1e-7,
// checked against float64 sin/cos by the GPU tests.
#pragma once

#include <hip/hip_runtime.h>

namespace hrf {

__device__ __forceinline__ void sincos_big(float x, float* s, float* c) {
  constexpr double kInvTwoPi = 0.15915494309189533577;  // 1 / (2 pi)
  const double t = static_cast<double>(x) * kInvTwoPi;
  const float rev = static_cast<float>(t - __builtin_rint(t));  // in [-0.5, 0.5]
  *s = __builtin_amdgcn_sinf(rev);
  *c = __builtin_amdgcn_cosf(rev);
}

// The same reduction without double precision, for the propagation's
// inner loops: 1/(2 pi) split into a float head kHi and tail kLo, the
// product x kHi rounded to hi with its exact rounding error
// e = fma(x, kHi, -hi), hi - rint(hi) exact (Sterbenz), and the revolution
// r = (hi - rint(hi)) + fma(x, kLo, e): for |x| below 2^21 revolutions'
// worth its error is the final rounding (2^-25 of a revolution) plus
// ~|x| 2^-48, the double-precision version's accuracy with six single-rate
// instructions instead of five at double rate.
__device__ __forceinline__ void sincos_big_ff(float x, float* s, float* c) {
  constexpr float kHi = 0.15915493667125701904f;        // float(1 / (2 pi))
  constexpr float kLo = 6.4206383167313347657e-09f;     // 1 / (2 pi) - kHi
  const float hi = x * kHi;
  const float e = fmaf(x, kHi, -hi);
  const float rev = (hi - __builtin_rintf(hi)) + fmaf(x, kLo, e);  // in [-0.5, 0.5]
  *s = __builtin_amdgcn_sinf(rev);
  *c = __builtin_amdgcn_cosf(rev);
}

}  // namespace hrf
