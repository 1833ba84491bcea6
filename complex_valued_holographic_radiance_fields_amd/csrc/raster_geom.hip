// raster_geom.hip — stage 1 (per-Gaussian projection, culling, radius, tile
// rectangle, render record) and the fused per-Gaussian geometry backward.
//
// One thread per Gaussian; everything the reference spreads over ~10
// launches, 4+6 cuBLAS batched GEMMs and an N-times repeated view matrix
// (forward.cu:221-294, forward_splat.cu:17-98, backward.cu:363-450,
// backward_splat.cu:364-417) is evaluated in registers.  Arithmetic order
// follows the reference source expression by expression (no contraction);
// the cuBLAS matmul chain is a left-to-right fmaf dot product over k.
#include "hrf_internal.h"

namespace hrf {
namespace {

// 3-term dot product in the fixed order fma(a2,b2, fma(a1,b1, a0*b0)).
__device__ __forceinline__ float dot3(float a0, float b0, float a1, float b1,
                                      float a2, float b2) {
  return fmaf(a2, b2, fmaf(a1, b1, a0 * b0));
}
__device__ __forceinline__ float dot2(float a0, float b0, float a1, float b1) {
  return fmaf(a1, b1, a0 * b0);
}

// float -> uint32 as the reference's (uint32_t) cast behaves on its target:
// truncation toward zero, negatives and NaN saturate to 0, overflow to max.
__device__ __forceinline__ uint32_t to_u32_sat(float f) {
  if (!(f > 0.0f)) return 0u;
  if (f >= 4294967296.0f) return 0xFFFFFFFFu;
  return static_cast<uint32_t>(f);
}

// Rotation in GLM column-major storage: R[c][r] = v[3c+r] with the nine
// values listed in forward.cu:41-45 (equal to the standard row-major
// rotation matrix entry (c,r)).  Quaternion normalised in-kernel first.
__device__ __forceinline__ void quat_rot(const float* q, float R[3][3]) {
  float r = q[0], x = q[1], y = q[2], z = q[3];
  const float norm = sqrtf(r * r + x * x + y * y + z * z);
  r /= norm;
  x /= norm;
  y /= norm;
  z /= norm;
  R[0][0] = 1.f - 2.f * (y * y + z * z);
  R[0][1] = 2.f * (x * y - r * z);
  R[0][2] = 2.f * (x * z + r * y);
  R[1][0] = 2.f * (x * y + r * z);
  R[1][1] = 1.f - 2.f * (x * x + z * z);
  R[1][2] = 2.f * (y * z - r * x);
  R[2][0] = 2.f * (x * z - r * y);
  R[2][1] = 2.f * (y * z + r * x);
  R[2][2] = 1.f - 2.f * (x * x + y * y);
}

// GLM mat3 product (type_mat3x3.inl:486-516):
// Res[c][r] = A[0][r]*B[c][0] + A[1][r]*B[c][1] + A[2][r]*B[c][2].
__device__ __forceinline__ void glm_mul(const float A[3][3], const float B[3][3],
                                        float Res[3][3]) {
#pragma unroll
  for (int c = 0; c < 3; ++c)
#pragma unroll
    for (int r = 0; r < 3; ++r)
      Res[c][r] = A[0][r] * B[c][0] + A[1][r] * B[c][1] + A[2][r] * B[c][2];
}

__device__ __forceinline__ void glm_diag(const float* s, float S[3][3]) {
#pragma unroll
  for (int c = 0; c < 3; ++c)
#pragma unroll
    for (int r = 0; r < 3; ++r) S[c][r] = 0.f;
  S[0][0] = s[0];
  S[1][1] = s[1];
  S[2][2] = s[2];
}

__device__ __forceinline__ void glm_transpose(const float A[3][3], float T[3][3]) {
#pragma unroll
  for (int c = 0; c < 3; ++c)
#pragma unroll
    for (int r = 0; r < 3; ++r) T[c][r] = A[r][c];
}

// Sigma row-major: sig[i][j] = GLM Sigma[i][j] with Sigma = transpose(SR)*SR
// (forward.cu:34-60).
__device__ __forceinline__ void cov3d(const float* q, const float* s, float sig[3][3]) {
  float R[3][3], S[3][3], SR[3][3], SRt[3][3], Sg[3][3];
  quat_rot(q, R);
  glm_diag(s, S);
  glm_mul(S, R, SR);
  glm_transpose(SR, SRt);
  glm_mul(SRt, SR, Sg);
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) sig[i][j] = Sg[i][j];
}

// Jacobian (forward.cu:64-122); returns false (J = 0) when clipped.
__device__ __forceinline__ bool jacobian(float tx, float ty, float tz, float fx,
                                         float fy, float lim_x, float lim_y,
                                         float near_plane, float far_plane,
                                         float J[2][3]) {
  if (tz <= near_plane || tz >= far_plane) {
    J[0][0] = J[0][1] = J[0][2] = J[1][0] = J[1][1] = J[1][2] = 0.f;
    return false;
  }
  const float tz2 = tz * tz;
  const float tx_tz = tx / tz;
  const float ty_tz = ty / tz;
  const float ctx = fminf(fmaxf(tx_tz, -lim_x), lim_x);
  const float cty = fminf(fmaxf(ty_tz, -lim_y), lim_y);
  const float cx = ctx * tz;
  const float cy = cty * tz;
  J[0][0] = fx / tz;
  J[0][1] = 0.0f;
  J[0][2] = -(fx * cx) / tz2;
  J[1][0] = 0.0f;
  J[1][1] = fy / tz;
  J[1][2] = -(fy * cy) / tz2;
  return true;
}

// cov2D chain ((J*W)*Sigma)*W^T*J^T (forward.cu:257-268) + 0.3 on the
// diagonal (forward.cu:283-287).  Also returns JW.
__device__ __forceinline__ void cov2d(const float J[2][3], const float Wm[3][3],
                                      const float sig[3][3], float JW[2][3],
                                      float cov[2][2]) {
  float M1[2][3], M2[2][3];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      JW[i][j] = dot3(J[i][0], Wm[0][j], J[i][1], Wm[1][j], J[i][2], Wm[2][j]);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      M1[i][j] = dot3(JW[i][0], sig[0][j], JW[i][1], sig[1][j], JW[i][2], sig[2][j]);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      M2[i][j] = dot3(M1[i][0], Wm[j][0], M1[i][1], Wm[j][1], M1[i][2], Wm[j][2]);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      cov[i][j] = dot3(M2[i][0], J[j][0], M2[i][1], J[j][1], M2[i][2], J[j][2]);
  cov[0][0] += 0.3f;
  cov[1][1] += 0.3f;
}

__global__ __launch_bounds__(256) void k_project(ProjectParams p) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= p.n) return;
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
    if (!culled) {
      const float mid = 0.5f * (ax + aw);
      const float disc = fmaxf(0.1f, mid * mid - det_cov);
      const float lambda1 = mid + sqrtf(disc);
      const float lambda2 = mid - sqrtf(disc);
      const float radius_f = ceilf(3.0f * sqrtf(fmaxf(lambda1, lambda2)));
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
  uint32_t bits = __float_as_uint(z);
  p.dkey[g] = (bits & 0x80000000u) ? (bits & 0x7FFFFFFFu) : (bits | 0x80000000u);
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
  // (forward_splat.cu:217-223), opacity, complex amplitude colour*e^{i phase}.
  const int RS = rec_stride(C);
  float* r = p.rec + g * RS;
  const float det = c_x * c_w - c_y * c_z;
  const float det_inv = 1.0f / det;
  float4 q0 = make_float4(mx, my, c_w * det_inv, -c_y * det_inv);
  float4 q1 = make_float4(-c_z * det_inv, c_x * det_inv, p.opac[g], 0.0f);
  reinterpret_cast<float4*>(r)[0] = q0;
  reinterpret_cast<float4*>(r)[1] = q1;
  float amp[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) amp[i] = 0.0f;
  for (int c = 0; c < C; ++c) {
    float sv, cvv;
    sincosf(p.phase[g * C + c], &sv, &cvv);
    const float col = p.colours[g * C + c];
    amp[2 * c] = col * cvv;
    amp[2 * c + 1] = col * sv;
  }
  reinterpret_cast<float4*>(r)[2] = make_float4(amp[0], amp[1], amp[2], amp[3]);
  if (rec_quads(C) > 3)
    reinterpret_cast<float4*>(r)[3] = make_float4(amp[4], amp[5], amp[6], amp[7]);
}

// ---------------------------------------------------------------- backward

__global__ __launch_bounds__(256) void k_geom_backward(GeomBwdParams p) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= p.n) return;
  const int C = p.C, P = p.P;
  const int AS = acc_stride(C, P);
  const float* a = p.acc + g * AS;
  const float tx = p.cam[g * 3 + 0], ty = p.cam[g * 3 + 1], tz = p.cam[g * 3 + 2];
  const bool clipped = (tz <= p.near_plane || tz >= p.far_plane);

  float Wm[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) Wm[i][j] = p.view[i * 3 + j];
  float J[2][3], sig[3][3], JW[2][3], cv[2][2];
  jacobian(tx, ty, tz, p.fx, p.fy, p.lim_x, p.lim_y, p.near_plane, p.far_plane, J);
  cov3d(p.quats + g * 4, p.scales + g * 3, sig);
  cov2d(J, Wm, sig, JW, cv);

  // grad means2D (accumulated by the render backward, already scaled by
  // (0.5W, 0.5H) as backward_splat.cu:160-161,275-276).
  const float gmx = a[0], gmy = a[1];
  // Conic gradients -> cov2D gradients with the reference's own map
  // (backward_splat.cu:285-296), applied to the per-Gaussian sums (the map
  // is linear in the conic gradients).
  const float dcx = a[2], dcy = a[3], dcz = a[4];
  float gxx = 0.f, gxy = 0.f, gyy = 0.f;
  if (dcx != 0.f || dcy != 0.f || dcz != 0.f) {
    const float cx = cv[0][0], cy = cv[0][1], cz = cv[1][0], cw = cv[1][1];
    const float det = cx * cw - cy * cz;
    const float di = 1.0f / det;
    const float a1 = cw * di * di;
    const float a2 = -cy * di * di;
    const float a3 = cx * di * di;
    gxx = dcx * a1 * cw + dcz * a2 * (-cy);
    gxy = dcx * a1 * (-cy) + dcy * (-di) + dcz * a2 * cx;
    gyy = dcx * a2 * (-cy) + dcz * a3 * cx;
  }
  const float G2[2][2] = {{gxx, gxy}, {gxy, gyy}};

  // means2D backward (backward.cu:453-497)
  float gcam0 = 0.f, gcam1 = 0.f, gcam2 = 0.f;
  if (!clipped) {
    const float z2 = tz * tz;
    gcam0 = -p.fx * gmx / tz;
    gcam1 = -p.fy * gmy / tz;
    gcam2 = (p.fx * tx * gmx / z2) + (p.fy * ty * gmy / z2);
  }

  // cov2D backward (backward.cu:426-439)
  float dC[2][3], dB[2][3], X[2][3], dSig[3][3], dA[2][3], dJ[2][3];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) dC[i][j] = dot2(G2[i][0], J[0][j], G2[i][1], J[1][j]);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      dB[i][j] = dot3(dC[i][0], Wm[0][j], dC[i][1], Wm[1][j], dC[i][2], Wm[2][j]);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) X[i][j] = dot2(G2[i][0], JW[0][j], G2[i][1], JW[1][j]);
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) dSig[i][j] = dot2(JW[0][i], X[0][j], JW[1][i], X[1][j]);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      dA[i][j] = dot3(dB[i][0], sig[j][0], dB[i][1], sig[j][1], dB[i][2], sig[j][2]);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      dJ[i][j] = dot3(dA[i][0], Wm[j][0], dA[i][1], Wm[j][1], dA[i][2], Wm[j][2]);

  // Jacobian backward (backward.cu:201-272): clamp mask, unclamped tx/ty.
  float jx = 0.f, jy = 0.f, jz = 0.f;
  if (!clipped) {
    const float tz2 = tz * tz;
    const float tz3 = tz2 * tz;
    const float tx_tz = tx / tz;
    const float ty_tz = ty / tz;
    const float xm = (tx_tz < -p.lim_x || tx_tz > p.lim_x) ? 0.0f : 1.0f;
    const float ym = (ty_tz < -p.lim_y || ty_tz > p.lim_y) ? 0.0f : 1.0f;
    const float dJ00_dtz = -p.fx / tz2;
    const float dJ02_dtx = xm * (-p.fx / tz2);
    const float dJ02_dtz = xm * (2.0f * p.fx * tx / tz3);
    const float dJ11_dtz = -p.fy / tz2;
    const float dJ12_dty = ym * (-p.fy / tz2);
    const float dJ12_dtz = ym * (2.0f * p.fy * ty / tz3);
    jx = dJ[0][2] * dJ02_dtx;
    jy = dJ[1][2] * dJ12_dty;
    jz = dJ[0][0] * dJ00_dtz + dJ[0][2] * dJ02_dtz + dJ[1][1] * dJ11_dtz +
         dJ[1][2] * dJ12_dtz;
  }
  p.g_cam[g * 3 + 0] = gcam0 + jx;
  p.g_cam[g * 3 + 1] = gcam1 + jy;
  p.g_cam[g * 3 + 2] = gcam2 + jz;
  p.g_z[g] = 0.0f;

  // Sigma backward in GLM storage (backward.cu:21-198).
  {
    const float* q = p.quats + g * 4;
    const float* s = p.scales + g * 3;
    float Gm[3][3];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) Gm[i][j] = dSig[i][j];  // G[i][j] = grad[i*3+j]
    float r = q[0], x = q[1], y = q[2], z = q[3];
    const float norm = sqrtf(r * r + x * x + y * y + z * z);
    r /= norm;
    x /= norm;
    y /= norm;
    z /= norm;
    float S[3][3], R[3][3];
    glm_diag(s, S);
    R[0][0] = 1.f - 2.f * (y * y + z * z);
    R[0][1] = 2.f * (x * y - r * z);
    R[0][2] = 2.f * (x * z + r * y);
    R[1][0] = 2.f * (x * y + r * z);
    R[1][1] = 1.f - 2.f * (x * x + z * z);
    R[1][2] = 2.f * (y * z - r * x);
    R[2][0] = 2.f * (x * z - r * y);
    R[2][1] = 2.f * (y * z + r * x);
    R[2][2] = 1.f - 2.f * (x * x + y * y);
    float dRr[3][3] = {{0.f, -2.f * z, 2.f * y}, {2.f * z, 0.f, -2.f * x}, {-2.f * y, 2.f * x, 0.f}};
    float dRx[3][3] = {{0.f, 2.f * y, 2.f * z}, {2.f * y, -4.f * x, -2.f * r}, {2.f * z, 2.f * r, -4.f * x}};
    float dRy[3][3] = {{-4.f * y, 2.f * x, 2.f * r}, {2.f * x, 0.f, 2.f * z}, {-2.f * r, 2.f * z, -4.f * y}};
    float dRz[3][3] = {{-4.f * z, -2.f * r, 2.f * x}, {2.f * r, -4.f * z, 2.f * y}, {2.f * x, 2.f * y, 0.f}};

    // temp = ((2 * transpose(R)) * G) * R
    float Rt2[3][3], T1[3][3], temp[3][3];
#pragma unroll
    for (int c = 0; c < 3; ++c)
#pragma unroll
      for (int rr = 0; rr < 3; ++rr) Rt2[c][rr] = 2.0f * R[rr][c];
    glm_mul(Rt2, Gm, T1);
    glm_mul(T1, R, temp);
    p.g_scale[g * 3 + 0] = temp[0][0] * s[0];
    p.g_scale[g * 3 + 1] = temp[1][1] * s[1];
    p.g_scale[g * 3 + 2] = temp[2][2] * s[2];

    float SR[3][3], Xr[3][3], Xx[3][3], Xy[3][3], Xz[3][3];
    glm_mul(S, R, SR);
    glm_mul(S, dRr, Xr);
    glm_mul(S, dRx, Xx);
    glm_mul(S, dRy, Xy);
    glm_mul(S, dRz, Xz);
    float gr = 0.f, gxq = 0.f, gyq = 0.f, gzq = 0.f;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        gr += Gm[i][j] * (Xr[j][i] * SR[i][j] + SR[j][i] * Xr[i][j]);
        gxq += Gm[i][j] * (Xx[j][i] * SR[i][j] + SR[j][i] * Xx[i][j]);
        gyq += Gm[i][j] * (Xy[j][i] * SR[i][j] + SR[j][i] * Xy[i][j]);
        gzq += Gm[i][j] * (Xz[j][i] * SR[i][j] + SR[j][i] * Xz[i][j]);
      }
    p.g_quat[g * 4 + 0] = gr;
    p.g_quat[g * 4 + 1] = gxq;
    p.g_quat[g * 4 + 2] = gyq;
    p.g_quat[g * 4 + 3] = gzq;
  }

  // Colour / phase from the per-Gaussian sums A_c = sum dcol*g_re,
  // B_c = sum dcol*g_im (backward_splat.cu:251-257 summed over pixels).
  for (int c = 0; c < C; ++c) {
    float sv, cvv;
    sincosf(p.phase[g * C + c], &sv, &cvv);
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
  hipLaunchKernelGGL(k_project, dim3(blocks_for(p.n, 256)), dim3(256), 0, s, p);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_geom_backward(const GeomBwdParams& p, hipStream_t s) {
  if (p.n == 0) return HRF_OK;
  hipLaunchKernelGGL(k_geom_backward, dim3(blocks_for(p.n, 256)), dim3(256), 0, s, p);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

}  // namespace hrf
