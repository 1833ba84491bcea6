// geom_math.h — per-Gaussian projection and geometry-backward arithmetic
// shared by the fused rasterizer kernels (raster_geom.hip) and the
// standalone geometry ops (geom_ops.hip).
//
// Arithmetic order follows the reference source expression by expression
// (built with -ffp-contract=off, so nothing is contracted); the cuBLAS
// matmul chains (forward.cu:265-268, backward.cu:426-439) are left-to-right
// fmaf dot products over k.  GLM matrices are column-major: A[c][r].
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace hrf {
namespace geom {

// 3-term dot product in the fixed order fma(a2,b2, fma(a1,b1, a0*b0)).
__device__ __forceinline__ float dot3(float a0, float b0, float a1, float b1,
                                      float a2, float b2) {
  return fmaf(a2, b2, fmaf(a1, b1, a0 * b0));
}
__device__ __forceinline__ float dot2(float a0, float b0, float a1, float b1) {
  return fmaf(a1, b1, a0 * b0);
}

// Division and square root: exact IEEE (kFast = false, the forward
// projection whose outputs are bit-exact) or the hardware reciprocal /
// square root (kFast = true, about 1 ulp: the fused raster backward, whose
// gradients only need fp32 accuracy).
template <bool kFast>
__device__ __forceinline__ float fdiv(float a, float b) {
  if constexpr (kFast) return a * __builtin_amdgcn_rcpf(b);
  else return a / b;
}
template <bool kFast>
__device__ __forceinline__ float fsqrt(float a) {
  if constexpr (kFast) return __builtin_amdgcn_sqrtf(a);
  else return sqrtf(a);
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
template <bool kFast = false>
__device__ __forceinline__ void quat_rot(const float* q, float R[3][3]) {
  float r = q[0], x = q[1], y = q[2], z = q[3];
  const float norm = fsqrt<kFast>(r * r + x * x + y * y + z * z);
  r = fdiv<kFast>(r, norm);
  x = fdiv<kFast>(x, norm);
  y = fdiv<kFast>(y, norm);
  z = fdiv<kFast>(z, norm);
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
template <bool kFast = false>
__device__ __forceinline__ void cov3d(const float* q, const float* s, float sig[3][3]) {
  float R[3][3], S[3][3], SR[3][3], SRt[3][3], Sg[3][3];
  quat_rot<kFast>(q, R);
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
template <bool kFast = false>
__device__ __forceinline__ bool jacobian(float tx, float ty, float tz, float fx,
                                         float fy, float lim_x, float lim_y,
                                         float near_plane, float far_plane,
                                         float J[2][3]) {
  if (tz <= near_plane || tz >= far_plane) {
    J[0][0] = J[0][1] = J[0][2] = J[1][0] = J[1][1] = J[1][2] = 0.f;
    return false;
  }
  const float tz2 = tz * tz;
  const float tx_tz = fdiv<kFast>(tx, tz);
  const float ty_tz = fdiv<kFast>(ty, tz);
  const float ctx = fminf(fmaxf(tx_tz, -lim_x), lim_x);
  const float cty = fminf(fmaxf(ty_tz, -lim_y), lim_y);
  const float cx = ctx * tz;
  const float cy = cty * tz;
  J[0][0] = fdiv<kFast>(fx, tz);
  J[0][1] = 0.0f;
  J[0][2] = fdiv<kFast>(-(fx * cx), tz2);
  J[1][0] = 0.0f;
  J[1][1] = fdiv<kFast>(fy, tz);
  J[1][2] = fdiv<kFast>(-(fy * cy), tz2);
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


// means2D backward (backward.cu:453-497): zero when clipped.
template <bool kFast = false>
__device__ __forceinline__ void means2d_bwd(float tx, float ty, float tz, float fx, float fy,
                                            float near_plane, float far_plane, float gmx,
                                            float gmy, float g[3]) {
  g[0] = g[1] = g[2] = 0.f;
  if (tz <= near_plane || tz >= far_plane) return;
  const float z2 = tz * tz;
  g[0] = fdiv<kFast>(-fx * gmx, tz);
  g[1] = fdiv<kFast>(-fy * gmy, tz);
  g[2] = fdiv<kFast>(fx * tx * gmx, z2) + fdiv<kFast>(fy * ty * gmy, z2);
}

// cov2D chain backward (backward.cu:426-439) for G2 = dL/dcov2D (2,2):
// dL_dC = G2 J, dL_dB = dL_dC W, dL_dSigma = JW^T (G2 JW),
// dL_dA = dL_dB Sigma^T, dL_dJ = dL_dA W^T.
__device__ __forceinline__ void cov2d_chain_bwd(const float G2[2][2], const float J[2][3],
                                                const float Wm[3][3], const float sig[3][3],
                                                const float JW[2][3], float dSig[3][3],
                                                float dJ[2][3]) {
  float dC[2][3], dB[2][3], X[2][3], dA[2][3];
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
}

// Jacobian backward (backward.cu:201-272): clamp mask on tx/tz, ty/tz, but
// the unclamped tx, ty in dJ02/dtz and dJ12/dtz; zero when clipped.
template <bool kFast = false>
__device__ __forceinline__ void jacobian_bwd(float tx, float ty, float tz, float fx, float fy,
                                             float lim_x, float lim_y, float near_plane,
                                             float far_plane, const float dJ[2][3],
                                             float g[3]) {
  g[0] = g[1] = g[2] = 0.f;
  if (tz <= near_plane || tz >= far_plane) return;
  const float tz2 = tz * tz;
  const float tz3 = tz2 * tz;
  const float tx_tz = fdiv<kFast>(tx, tz);
  const float ty_tz = fdiv<kFast>(ty, tz);
  const float xm = (tx_tz < -lim_x || tx_tz > lim_x) ? 0.0f : 1.0f;
  const float ym = (ty_tz < -lim_y || ty_tz > lim_y) ? 0.0f : 1.0f;
  const float dJ00_dtz = fdiv<kFast>(-fx, tz2);
  const float dJ02_dtx = xm * fdiv<kFast>(-fx, tz2);
  const float dJ02_dtz = xm * fdiv<kFast>(2.0f * fx * tx, tz3);
  const float dJ11_dtz = fdiv<kFast>(-fy, tz2);
  const float dJ12_dty = ym * fdiv<kFast>(-fy, tz2);
  const float dJ12_dtz = ym * fdiv<kFast>(2.0f * fy * ty, tz3);
  g[0] = dJ[0][2] * dJ02_dtx;
  g[1] = dJ[1][2] * dJ12_dty;
  g[2] = dJ[0][0] * dJ00_dtz + dJ[0][2] * dJ02_dtz + dJ[1][1] * dJ11_dtz + dJ[1][2] * dJ12_dtz;
}

// Sigma backward in GLM storage (backward.cu:21-198) for Gm[i][j] =
// dL/dSigma[i*3+j]: grad_s[k] = (2 R^T G R)[k][k] * s[k]; grad_q by the
// reference's elementwise (Hadamard) sums over S * dR/dq (the quaternion is
// normalised again without a chain through the normalisation).
template <bool kFast = false>
__device__ __forceinline__ void cov3d_bwd(const float Gm[3][3], const float* q, const float* s,
                                          float gq[4], float gs[3]) {
  float r = q[0], x = q[1], y = q[2], z = q[3];
  const float norm = fsqrt<kFast>(r * r + x * x + y * y + z * z);
  r = fdiv<kFast>(r, norm);
  x = fdiv<kFast>(x, norm);
  y = fdiv<kFast>(y, norm);
  z = fdiv<kFast>(z, norm);
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
  gs[0] = temp[0][0] * s[0];
  gs[1] = temp[1][1] * s[1];
  gs[2] = temp[2][2] * s[2];

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
  gq[0] = gr;
  gq[1] = gxq;
  gq[2] = gyq;
  gq[3] = gzq;
}

}  // namespace geom
}  // namespace hrf
