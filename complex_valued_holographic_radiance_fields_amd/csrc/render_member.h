// render_member.h — the forward render's per-member compositing step for
// its fast loop (k_render_fwd), shared with the VALU calibration kernel of
// the tests (which runs the same loop body over staged members of known
// count to measure the issue rate this instruction mix reaches).
#pragma once

#include "hrf_internal.h"

namespace hrf {

// Forward member evaluation (fast loop: staged conics that cannot round to
// a positive exponent, so the reference's "power > 0: skip" test is not
// evaluated).  The exponent is in base 2 with log2(o w) folded in, as a
// quadratic in the pixel's offset (u, v) from the tile centre:
// pw = c0 + u (c1 + c3 u + c4 v) + v (c2 + c5 v), five fused multiply-adds
// (the staging forms c0..c5 from the mean, the conic scaled by
// kc = -log2(e)/2 and log2(o w); |u|, |v| <= 7.5, so the terms stay within
// a few times the exponent's own size), and alpha = min(0.99, exp2(pw)).
// A lane is done exactly when T < 1e-4 (T changes only on composited
// members, and a lane stops at the member that takes T below 1e-4; lanes
// outside the image start at T = 0), so no separate flag is carried.
// Branch-free: lanes that are done take alpha = 0, which leaves T and the
// field exactly unchanged.  `evaluated` counts the members evaluated while
// the lane was live (one add of the live mask, no index select): a lane
// composites every member until the one that ends it, so the count minus
// one is that member's index.  Staged record quads: a = (c0, c1, c2, c3),
// b = (c4, c5, re0, im0), c = (re1, im1, re2, im2) (C >= 2).
// The quadratic's coefficients for a member with mean (mx, my), scaled
// conic (qa, qb, qc) (exponent qa dx^2 + qb dx dy + qc dy^2 + lw in the
// offsets dx, dy from the mean) about the tile centre (xc, yc): with
// M = mean - centre, c0 = M.x (qa M.x + qb M.y) + qc M.y^2 + lw (the
// exponent at the centre), c1 = -(2 qa M.x + qb M.y), c2 = -(qb M.x + 2 qc
// M.y); the exponent at offset (u, v) from the centre is then
// c0 + u (c1 + qa u + qb v) + v (c2 + qc v) (quad_exponent).
__device__ __forceinline__ void quad_coeffs(float mx, float my, float qa, float qb, float qc,
                                            float lw, float xc, float yc, float* c0, float* c1,
                                            float* c2) {
  const float ax = mx - xc, ay = my - yc;
  *c0 = fmaf(ax, fmaf(qa, ax, qb * ay), fmaf(qc * ay, ay, lw));
  *c1 = -fmaf(2.0f * qa, ax, qb * ay);
  *c2 = -fmaf(qb, ax, (2.0f * qc) * ay);
}
__device__ __forceinline__ float quad_exponent(float c0, float c1, float c2, float qa, float qb,
                                               float qc, float u, float v) {
  const float t1 = fmaf(qb, v, fmaf(qa, u, c1));
  const float t2 = fmaf(qc, v, c2);
  return fmaf(v, t2, fmaf(u, t1, c0));
}

// kClamp false: the batch's members have o w small enough that exp2(pw)
// stays below kMaxAlpha, and the clamp is left out (same result).
template <int C, bool kClamp = true>
__device__ __forceinline__ void fwd_member(const float4 a, const float4 b, const float4 c,
                                           float u, float v, float& T,
                                           float (&acc)[2 * C], int& evaluated) {
  const float pw = quad_exponent(a.x, a.y, a.z, a.w, b.x, b.y, u, v);
  const bool live = !(T < kTermT);
  const float e = __builtin_amdgcn_exp2f(pw);
  const float alpha = live ? (kClamp ? fminf(kMaxAlpha, e) : e) : 0.0f;
  const float sT = alpha * T;
  const float amp[6] = {b.z, b.w, c.x, c.y, c.z, c.w};
#pragma unroll
  for (int k = 0; k < C; ++k) {
    acc[2 * k] = fmaf(sT, amp[2 * k], acc[2 * k]);
    acc[2 * k + 1] = fmaf(sT, amp[2 * k + 1], acc[2 * k + 1]);
  }
  // The reference's rounding: 1 - alpha rounded first (forward_splat.cu:237);
  // the exactly rounded T - alpha T differs from it in the last bit.
  T = T * (1.0f - alpha);
  evaluated += live ? 1 : 0;
}

}  // namespace hrf
