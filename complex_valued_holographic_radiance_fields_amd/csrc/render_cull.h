// render_cull.h — the render kernels' exact culling tests, shared with the
// pair emission, which tags each (tile, gaussian) pair of large sorts with
// the forward's visibility test so that the forward can skip the invisible
// entries of its tile lists without gathering their records.
#pragma once

#include "hrf_internal.h"

namespace hrf {

// Culling of backward work.  A Gaussian can reach alpha >= 1/255 at a pixel
// only where q = d^T A d <= 2 ln(255 o w) (power = -q/2, A the conic,
// d = mean - pixel).  alpha_threshold returns that bound widened by 0.1% +
// 0.01, far beyond the rounding of the exp/power evaluation, or -1 when no
// pixel can qualify (o*w below 1/255).
__device__ __forceinline__ float alpha_threshold(float ow) {
  if (ow * 255.0f < 0.999f) return -1.0f;
  return 2.0f * __logf(ow * 255.0f) * 1.001f + 0.01f;
}

// Cull tests.  q(d) = cxx dx^2 + 2 cxy dx dy + czz dy^2 with d = mean -
// pixel centre: a convex quadratic when the conic is positive definite.
// CullShape holds the conic with 2 cxy and the two 1-D minimiser slopes
// -cxy/cxx and -cxy/czz (hardware reciprocals).  pd = false (not positive
// definite, or NaN): never culled.
struct CullShape {
  float cxx, czz, t12, nx, nz;
  bool pd;
};

__device__ __forceinline__ CullShape cull_shape(float cxx, float cxy, float czz) {
  CullShape c;
  c.cxx = cxx;
  c.czz = czz;
  c.t12 = 2.0f * cxy;
  c.pd = cxx > 0.0f && czz > 0.0f && cxx * czz - cxy * cxy > 0.0f;
  c.nx = -cxy * __builtin_amdgcn_rcpf(cxx);
  c.nz = -cxy * __builtin_amdgcn_rcpf(czz);
  return c;
}

// min of q(u, v) = a u^2 + t u v + b v^2 over u in [lo, hi] at a fixed v:
// the 1-D minimiser n v (n = -t / 2a), clamped to the interval.  q at any
// point of the interval bounds the minimum from above, and the minimiser's
// rounding moves q by a (du)^2, far inside the thresholds' margins.
__device__ __forceinline__ float seg_min(float a, float b, float t, float n, float v, float lo,
                                         float hi) {
  const float u = fminf(fmaxf(n * v, lo), hi);
  return fmaf(u, fmaf(a, u, t * v), (b * v) * v);
}

// Minimum of q over the box of pixel centres [x0, x0+ext] x [y0, y0+ext]
// (0 when the mean lies in it).  A convex function's minimum over a box is
// reached on the faces the mean lies beyond: the segment from the mean (q's
// minimum) to any point of the box enters the box through one of them, and
// q along it never exceeds its value at that point.  So it is the smaller
// of the minima over the face x = clamp(mx, x0, x1) (over the box's dy
// range) and the face y = clamp(my, y0, y1) (over its dx range); when the
// mean lies within the box's range of a coordinate, that "face" is a line
// through the box, whose minimum only bounds the box's from above.
__device__ __forceinline__ float box_min(float mx, float my, const CullShape& c, float x0,
                                         float y0, float ext) {
  const float dxl = mx - (x0 + ext), dxh = mx - x0;
  const float dyl = my - (y0 + ext), dyh = my - y0;
  const float dxn = fminf(fmaxf(0.0f, dxl), dxh);  // mx - clamp(mx, x0, x1)
  const float dyn = fminf(fmaxf(0.0f, dyl), dyh);
  const float mv = seg_min(c.czz, c.cxx, c.t12, c.nz, dxn, dyl, dyh);
  const float mh = seg_min(c.cxx, c.czz, c.t12, c.nx, dyn, dxl, dxh);
  return fminf(mv, mh);
}

// Exact test: does q(d) <= thr hold at some point of that box?
__device__ __forceinline__ bool box_reaches(float mx, float my, const CullShape& c, float thr,
                                            float x0, float y0, float ext) {
  return !c.pd || box_min(mx, my, c, x0, y0, ext) <= thr;
}

// Forward members without effect.  A Gaussian whose alpha stays below 2^-26
// at every pixel of the tile (q > 2 ln(o w 2^26) over the tile's pixel
// centres, widened as above) cannot change T there: alpha T is below half
// an ulp of T, so T (1 - alpha) rounds back to T (1 - alpha rounds to 1), and
// the termination test and
// final_T are exactly as if it had been composited.  Its field contribution
// is below 2^-25 T |amplitude|.  Such members are not staged; the tile's
// largest such list position still counts as the last contributor for
// pixels that never terminate (every culled member has power <= 0 there, as
// a composited one would).  Non-positive-definite conics are never culled.
__device__ __forceinline__ float invisible_threshold(float ow) {
  const float thr = 2.0f * __logf(ow * 67108864.0f);  // alpha < 2^-26
  return fmaxf(thr, 0.0f) * 1.001f + 0.01f;
}

// Pair tags of large sorts.  The forward culls the members of a (tile,
// plane) list whose alpha stays below 2^-26 over the tile (box_reaches with
// invisible_threshold of the plane's o w).  The pair emission makes that
// test once per (tile, gaussian) pair for all of the gaussian's planes at
// once, against the largest of their thresholds: a pair it rejects would be
// culled in every plane.  A CullKey holds the test's per-gaussian inputs as
// two quads, (mx, my, cxx, czz) and (2 cxy, nx, nz, thr): thr is +inf for a
// conic that is not positive definite (never culled) and -inf for a
// gaussian in no plane (no list member).
struct CullKey {
  float4 a, b;
};

// q0, q1: the render record's first two quads (mx, my, i00, i01) and
// (i10, i11, o, 1/det); w: the gaussian's P plane weights.
__device__ __forceinline__ CullKey cull_key(const float4 q0, const float4 q1, const float* w,
                                            int P) {
  const CullShape c = cull_shape(q0.z, q0.w, q1.y);
  float thr = -__builtin_inff();
  for (int p = 0; p < P; ++p) {
    const float wp = w[p];
    if (!(wp < kPlaneCutoff)) thr = fmaxf(thr, invisible_threshold(q1.z * wp));
  }
  if (!c.pd && thr > -__builtin_inff()) thr = __builtin_inff();
  CullKey k;
  k.a = make_float4(q0.x, q0.y, c.cxx, c.czz);
  k.b = make_float4(c.t12, c.nx, c.nz, thr);
  return k;
}

// Does some plane's forward keep this gaussian in the tile whose pixel
// centres start at (tx0, ty0)?  (NaN box minima keep it, as box_reaches
// does through its positive-definite test.)
__device__ __forceinline__ bool pair_visible(const CullKey& k, float tx0, float ty0) {
  CullShape c;
  c.cxx = k.a.z;
  c.czz = k.a.w;
  c.t12 = k.b.x;
  c.nx = k.b.y;
  c.nz = k.b.z;
  c.pd = true;
  return !(box_min(k.a.x, k.a.y, c, tx0, ty0, static_cast<float>(kTile - 1)) > k.b.w);
}

}  // namespace hrf
