// raster_geom.hip — stage 1 (per-Gaussian projection, culling, radius, tile
// rectangle, render record) and the fused per-Gaussian geometry backward.
//
// One thread per Gaussian; everything the reference spreads over ~10
// launches, 4+6 cuBLAS batched GEMMs and an N-times repeated view matrix
// (forward.cu:221-294, forward_splat.cu:17-98, backward.cu:363-450,
// backward_splat.cu:364-417) is evaluated in registers.  Arithmetic order
// follows the reference source expression by expression (no contraction);
// the cuBLAS matmul chain is a left-to-right fmaf dot product over k.
#include "geom_math.h"
#include "fast_trig.h"
#include "hrf_internal.h"

namespace hrf {
namespace {

using namespace geom;


__device__ __forceinline__ uint32_t depth_key(float z) {
  const uint32_t bits = __float_as_uint(z);
  return (bits & 0x80000000u) ? (bits & 0x7FFFFFFFu) : (bits | 0x80000000u);
}

// Returns whether g's depth key is below its predecessor's.
__device__ __forceinline__ bool project_one(const ProjectParams& p, int64_t g) {
  const int C = p.C, P = p.P;
  const float tx = p.cam[g * 3 + 0], ty = p.cam[g * 3 + 1], tz = p.cam[g * 3 + 2];
  const float z = p.z[g];

  // means2D (forward.cu:297-330)
  float mx, my;
  if (tz <= p.near_plane || tz >= p.far_plane) {
    mx = 1e6f;
    my = 1e6f;
  } else {
    const float inv_z = 1.0f / tz;
    const float px_div = -tx * inv_z;
    const float py_div = -ty * inv_z;
    mx = p.fx * px_div + p.px;
    my = p.fy * py_div + p.py;
  }

  float Wm[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) Wm[i][j] = p.view[i * 3 + j];

  float J[2][3], sig[3][3], JW[2][3], cv[2][2];
  jacobian(tx, ty, tz, p.fx, p.fy, p.lim_x, p.lim_y, p.near_plane, p.far_plane, J);
  cov3d(p.quats + g * 4, p.scales + g * 3, sig);
  cov2d(J, Wm, sig, JW, cv);
  const float c_x = cv[0][0], c_y = cv[0][1], c_z = cv[1][0], c_w = cv[1][1];

  // Culling, eigen-radius and tile rectangle (forward_splat.cu:17-98,
  // auxiliary.h:119-137); antialiasing is always on (rasterizer_splat.cu:422).
  uint32_t tiles = 0;
  uint2 rect = make_uint2(0u, 0u);
  bool culled = (z <= p.near_plane || z >= p.far_plane);
  if (!culled) {
    float ax = c_x, ay = c_y, az = c_z, aw = c_w;
    float det_cov = ax * aw - ay * az;
    if (fabsf(det_cov) < 1e-10f) {
      culled = true;
    } else {
      ax += 0.3f;
      aw += 0.3f;
      det_cov = ax * aw - ay * az;
      if (fabsf(det_cov) < 1e-8f) culled = true;
    }
    float radius_f = 0.0f;
    if (!culled) {
      const float mid = 0.5f * (ax + aw);
      const float disc = fmaxf(0.1f, mid * mid - det_cov);
      const float lambda1 = mid + sqrtf(disc);
      const float lambda2 = mid - sqrtf(disc);
      radius_f = ceilf(3.0f * sqrtf(fmaxf(lambda1, lambda2)));
      // A NaN or non-positive radius (a degenerate covariance: zero
      // quaternion, NaN or infinite scale; undefined in the reference)
      // culls the Gaussian, so it reaches no tile list; so does a NaN 2-D
      // mean (NaN camera-space x or y, whose covariance the Jacobian's clamp
      // keeps finite), which would otherwise land in tile 0 and composite
      // with alpha fminf(0.99, NaN) = 0.99.
      if (!(radius_f > 0.0f) || isnan(mx) || isnan(my)) culled = true;
    }
    if (!culled) {
      const int rad_i = radius_f < 2147483520.0f ? static_cast<int>(radius_f) : 2147483520;
      const int radius = rad_i > 1 ? rad_i : 1;
      const float rf = static_cast<float>(radius);
      const uint32_t gx = static_cast<uint32_t>(p.gx), gy = static_cast<uint32_t>(p.gy);
      uint32_t minx = to_u32_sat((mx - rf) / 16.0f);
      uint32_t miny = to_u32_sat((my - rf) / 16.0f);
      minx = minx < gx - 1 ? minx : gx - 1;
      miny = miny < gy - 1 ? miny : gy - 1;
      uint32_t maxx = to_u32_sat(((mx + rf) + 16.0f - 1.0f) / 16.0f);
      uint32_t maxy = to_u32_sat(((my + rf) + 16.0f - 1.0f) / 16.0f);
      maxx = maxx > 1u ? maxx : 1u;
      maxy = maxy > 1u ? maxy : 1u;
      maxx = maxx < gx ? maxx : gx;
      maxy = maxy < gy ? maxy : gy;
      if (maxx <= minx) maxx = (minx + 1 < gx) ? minx + 1 : gx;
      if (maxy <= miny) maxy = (miny + 1 < gy) ? miny + 1 : gy;
      tiles = (maxy - miny) * (maxx - minx);
      rect = make_uint2(minx | (miny << 16), maxx | (maxy << 16));
    }
  }
  p.tiles[g] = tiles;
  p.rect[g] = rect;

  // Depth key (rasterizer_splat.cu:150-158): ascending key == front to back.
  const uint32_t dk = depth_key(z);
  p.dkey[g] = dk;
  // Keys already non-decreasing (the reference's caller sorts by depth)
  // make the stable depth sort the identity; it then skips itself.
  const bool unsorted = p.part_t && g > 0 && depth_key(p.z[g - 1]) > dk;
  // Visibility: defined as 0.2 < z_cam and near < z_cam < far (the
  // reference's checkFrustum reads its 3x3 matrix out of bounds).
  p.vis[g] = (tz > 0.2f && tz > p.near_plane && tz < p.far_plane) ? 1u : 0u;

  // Plane membership: a plane is skipped when w < 1e-6 (forward_splat.cu:208).
  uint32_t mask = 0;
  for (int q = 0; q < P; ++q) {
    const float w = p.pprobs[g * P + q];
    if (!(w < kPlaneCutoff)) mask |= (1u << q);
  }
  p.pmask[g] = mask;

  // Render record: conic as the render kernels evaluate it
  // (forward_splat.cu:217-223), opacity, 1/det (for the backward's
  // conic-to-covariance gradient map), complex amplitude colour*e^{i phase}.
  const int RS = rec_stride(C);
  float* r = p.rec + g * RS;
  const float det = c_x * c_w - c_y * c_z;
  const float det_inv = 1.0f / det;
  float4 q0 = make_float4(mx, my, c_w * det_inv, -c_y * det_inv);
  float4 q1 = make_float4(-c_z * det_inv, c_x * det_inv, p.opac[g], det_inv);
  reinterpret_cast<float4*>(r)[0] = q0;
  reinterpret_cast<float4*>(r)[1] = q1;
  float amp[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) amp[i] = 0.0f;
  for (int c = 0; c < C; ++c) {
    float sv, cvv;  // a few 1e-7 absolute for any phase: the amplitude to fp32 accuracy
    sincos_big(p.phase[g * C + c], &sv, &cvv);
    const float col = p.colours[g * C + c];
    amp[2 * c] = col * cvv;
    amp[2 * c + 1] = col * sv;
  }
  reinterpret_cast<float4*>(r)[2] = make_float4(amp[0], amp[1], amp[2], amp[3]);
  if (rec_quads(C) > 3)
    reinterpret_cast<float4*>(r)[3] = make_float4(amp[4], amp[5], amp[6], amp[7]);
  return unsorted;
}

// One thread per Gaussian.  With part_t set, each block also leaves the sums
// of its Gaussians' tile counts and visibility flags (kProjThreads-Gaussian
// blocks: the granularity the pair emission and the visible compaction scan
// at), so the offsets need no separate pass over the counts.
__global__ __launch_bounds__(kProjThreads) void k_project(ProjectParams p) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  for (int64_t e = g; e < p.zero_n; e += static_cast<int64_t>(gridDim.x) * kProjThreads)
    p.zero[e] = 0;
  const bool unsorted = g < p.n && project_one(p, g);
  if (p.part_t) {
    __shared__ uint64_t s_t[kProjThreads / 64];
    __shared__ uint32_t s_v[kProjThreads / 64];
    uint64_t t = g < p.n ? p.tiles[g] : 0u;
    uint32_t v = g < p.n ? p.vis[g] : 0u;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      t += __shfl_xor(t, d, 64);
      v += __shfl_xor(v, d, 64);
    }
    if ((threadIdx.x & 63) == 0) {
      s_t[threadIdx.x >> 6] = t;
      s_v[threadIdx.x >> 6] = v;
    }
    const bool any_unsorted = __syncthreads_or(unsorted ? 1 : 0) != 0;
    if (threadIdx.x == 0) {
      uint64_t a = 0;
      uint32_t b = 0;
#pragma unroll
      for (int w = 0; w < kProjThreads / 64; ++w) {
        a += s_t[w];
        b += s_v[w];
      }
      // The visible count (at most kProjThreads) carries the block's
      // depth-order flag in bit 31.
      p.part_t[blockIdx.x] = a;
      p.part_v[blockIdx.x] = b | (any_unsorted ? kPartFlag : 0u);
    }
  }
}

// ---------------------------------------------------------------- backward

// The accumulator records of a block's kGeomBwdThreads Gaussians are one
// contiguous run of words: it is staged into LDS with consecutive lanes on
// consecutive words (kAccUnroll loads in flight per thread), then each
// thread reads its own record (LDS record stride padded to odd).
constexpr int kGeomBwdThreads = 256;
constexpr int kAccUnroll = 8;

__global__ __launch_bounds__(kGeomBwdThreads) void k_geom_backward(GeomBwdParams p) {
  extern __shared__ float s_acc[];
  const int C = p.C, P = p.P;
  const int AS = acc_stride(C, P);
  const int ASP = AS | 1;
  {
    const int64_t g0 = static_cast<int64_t>(blockIdx.x) * kGeomBwdThreads;
    const int64_t rows = p.n - g0 < kGeomBwdThreads ? p.n - g0 : kGeomBwdThreads;
    const float* src = p.acc + g0 * AS;
    const int cnt = static_cast<int>(rows) * AS;
    // (row, column) of word e, stepped by kGeomBwdThreads words per load
    const int dq = kGeomBwdThreads / AS, dm = kGeomBwdThreads - dq * AS;
    int r = static_cast<int>(threadIdx.x) / AS;
    int c = static_cast<int>(threadIdx.x) - r * AS;
    for (int e0 = threadIdx.x; e0 < cnt; e0 += kAccUnroll * kGeomBwdThreads) {
      float v[kAccUnroll];
#pragma unroll
      for (int u = 0; u < kAccUnroll; ++u) {
        const int e = e0 + u * kGeomBwdThreads;
        v[u] = e < cnt ? src[e] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < kAccUnroll; ++u) {
        if (e0 + u * kGeomBwdThreads < cnt) s_acc[r * ASP + c] = v[u];
        r += dq;
        c += dm;
        if (c >= AS) {
          c -= AS;
          ++r;
        }
      }
    }
  }
  __syncthreads();
  const int64_t g = static_cast<int64_t>(blockIdx.x) * kGeomBwdThreads + threadIdx.x;
  if (g >= p.n) return;
  const float* a = s_acc + threadIdx.x * ASP;
  const float tx = p.cam[g * 3 + 0], ty = p.cam[g * 3 + 1], tz = p.cam[g * 3 + 2];

  float Wm[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) Wm[i][j] = p.view[i * 3 + j];
  float J[2][3], sig[3][3], JW[2][3], cv[2][2];
  jacobian<true>(tx, ty, tz, p.fx, p.fy, p.lim_x, p.lim_y, p.near_plane, p.far_plane, J);
  cov3d<true>(p.quats + g * 4, p.scales + g * 3, sig);
  cov2d(J, Wm, sig, JW, cv);

  // grad means2D (accumulated by the render backward, already scaled by
  // (0.5W, 0.5H) as backward_splat.cu:160-161,275-276).
  const float gmx = a[0], gmy = a[1];
  // cov2D gradients: the render backward already applied the reference's
  // conic-to-covariance map (backward_splat.cu:285-296), per pixel or per
  // block, before the sums reached these records.
  const float G2[2][2] = {{a[2], a[3]}, {a[3], a[4]}};

  float gm[3], dSig[3][3], dJ[2][3], gj[3];
  means2d_bwd<true>(tx, ty, tz, p.fx, p.fy, p.near_plane, p.far_plane, gmx, gmy, gm);
  cov2d_chain_bwd(G2, J, Wm, sig, JW, dSig, dJ);
  jacobian_bwd<true>(tx, ty, tz, p.fx, p.fy, p.lim_x, p.lim_y, p.near_plane, p.far_plane, dJ, gj);
  p.g_cam[g * 3 + 0] = gm[0] + gj[0];
  p.g_cam[g * 3 + 1] = gm[1] + gj[1];
  p.g_cam[g * 3 + 2] = gm[2] + gj[2];
  p.g_z[g] = 0.0f;

  float gq[4], gs[3];
  cov3d_bwd<true>(dSig, p.quats + g * 4, p.scales + g * 3, gq, gs);
#pragma unroll
  for (int i = 0; i < 4; ++i) p.g_quat[g * 4 + i] = gq[i];
#pragma unroll
  for (int i = 0; i < 3; ++i) p.g_scale[g * 3 + i] = gs[i];

  // Colour / phase from the per-Gaussian sums A_c = sum dcol*g_re,
  // B_c = sum dcol*g_im (backward_splat.cu:251-257 summed over pixels).
  for (int c = 0; c < C; ++c) {
    float sv, cvv;  // a few 1e-7 absolute for any phase: ample for gradients
    sincos_big(p.phase[g * C + c], &sv, &cvv);
    const float A = a[5 + c], B = a[5 + C + c];
    const float col = p.colours[g * C + c];
    p.g_col[g * C + c] = cvv * A + sv * B;
    p.g_phase[g * C + c] = col * (-sv * A + cvv * B);
  }
  // Opacity / plane from Q_p = sum G*dL_dalpha (backward_splat.cu:299-300).
  const float o = p.opac[g];
  float go = 0.f;
  for (int q = 0; q < P; ++q) {
    const float Q = a[5 + 2 * C + q];
    const float w = p.pprobs[g * P + q];
    go += w * Q;
    p.g_plane[g * P + q] = o * Q;
  }
  p.g_opac[g] = go;
}

}  // namespace

int launch_project(const ProjectParams& p, hipStream_t s) {
  if (p.n == 0) return HRF_OK;
  hipLaunchKernelGGL(k_project, dim3(blocks_for(p.n, kProjThreads)), dim3(kProjThreads), 0, s,
                     p);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_geom_backward(const GeomBwdParams& p, hipStream_t s) {
  if (p.n == 0) return HRF_OK;
  const size_t lds = static_cast<size_t>(kGeomBwdThreads) * (acc_stride(p.C, p.P) | 1) *
                    sizeof(float);
  hipLaunchKernelGGL(k_geom_backward, dim3(blocks_for(p.n, kGeomBwdThreads)),
                     dim3(kGeomBwdThreads), lds, s, p);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

}  // namespace hrf
