// geom_ops.hip — the reference's standalone per-Gaussian geometry operators
// (compute_cov3d / jacobian / cov2d / means2d / invert_cov2d, forward and
// backward), each one thread per Gaussian on the caller's stream.
//
// The rasterizer itself never calls these: its projection and geometry
// backward are fused into k_project / k_geom_backward.  They exist because
// the reference exposes them as separate autograd operators
// (python_import.py:53-281, binding.cpp:14-25) and its Python splat path
// calls them; they share geom_math.h with the fused kernels, so both give
// the same bits.
#include "geom_math.h"
#include "hrf_internal.h"

namespace hrf {
namespace {

using namespace geom;

struct Cam {
  float fx, fy, px, py, lim_x, lim_y, near_plane, far_plane;
};

Cam make_cam(float fx, float fy, float px, float py, int width, int height, float near_plane,
             float far_plane) {
  Cam c;
  c.fx = fx;
  c.fy = fy;
  c.px = px;
  c.py = py;
  // half_tan_fov = 0.5f * width / fx (forward.cu:199-200), lim = 1.3f * it
  // (forward.cu:93-94, backward.cu:227-228).
  const float htx = 0.5f * static_cast<float>(width) / fx;
  const float hty = 0.5f * static_cast<float>(height) / fy;
  c.lim_x = 1.3f * htx;
  c.lim_y = 1.3f * hty;
  c.near_plane = near_plane;
  c.far_plane = far_plane;
  return c;
}

__device__ __forceinline__ void load33(const float* a, float m[3][3]) {
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) m[i][j] = a[i * 3 + j];
}
__device__ __forceinline__ void load23(const float* a, float m[2][3]) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) m[i][j] = a[i * 3 + j];
}

__global__ __launch_bounds__(256) void k_cov3d_fwd(const float* __restrict__ q,
                                                   const float* __restrict__ s, int64_t n,
                                                   float* __restrict__ out) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n) return;
  float sig[3][3];
  cov3d(q + g * 4, s + g * 3, sig);
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) out[g * 9 + i * 3 + j] = sig[i][j];
}

__global__ __launch_bounds__(256) void k_cov3d_bwd(const float* __restrict__ grad,
                                                   const float* __restrict__ q,
                                                   const float* __restrict__ s, int64_t n,
                                                   float* __restrict__ gq,
                                                   float* __restrict__ gs) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n) return;
  float Gm[3][3], dq[4], ds[3];
  load33(grad + g * 9, Gm);
  cov3d_bwd(Gm, q + g * 4, s + g * 3, dq, ds);
#pragma unroll
  for (int i = 0; i < 4; ++i) gq[g * 4 + i] = dq[i];
#pragma unroll
  for (int i = 0; i < 3; ++i) gs[g * 3 + i] = ds[i];
}

__global__ __launch_bounds__(256) void k_jacobian_fwd(const float* __restrict__ cam, int64_t n,
                                                      Cam c, float* __restrict__ out) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n) return;
  float J[2][3];
  jacobian(cam[g * 3 + 0], cam[g * 3 + 1], cam[g * 3 + 2], c.fx, c.fy, c.lim_x, c.lim_y,
           c.near_plane, c.far_plane, J);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) out[g * 6 + i * 3 + j] = J[i][j];
}

__global__ __launch_bounds__(256) void k_jacobian_bwd(const float* __restrict__ grad,
                                                      const float* __restrict__ cam, int64_t n,
                                                      Cam c, float* __restrict__ gcam) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n) return;
  float dJ[2][3], gj[3];
  load23(grad + g * 6, dJ);
  jacobian_bwd(cam[g * 3 + 0], cam[g * 3 + 1], cam[g * 3 + 2], c.fx, c.fy, c.lim_x, c.lim_y,
               c.near_plane, c.far_plane, dJ, gj);
#pragma unroll
  for (int i = 0; i < 3; ++i) gcam[g * 3 + i] = gj[i];
}

// compute_cov2d_forward (forward.cu:221-294): cov2D + the saved J, Sigma,
// the view matrix repeated per Gaussian, and JW.
__global__ __launch_bounds__(256) void k_cov2d_fwd(const float* __restrict__ cam,
                                                   const float* __restrict__ q,
                                                   const float* __restrict__ s,
                                                   const float* __restrict__ view, int64_t n,
                                                   Cam c, float* __restrict__ cov_out,
                                                   float* __restrict__ J_out,
                                                   float* __restrict__ sig_out,
                                                   float* __restrict__ W_out,
                                                   float* __restrict__ JW_out) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n) return;
  float Wm[3][3], J[2][3], sig[3][3], JW[2][3], cv[2][2];
  load33(view, Wm);
  jacobian(cam[g * 3 + 0], cam[g * 3 + 1], cam[g * 3 + 2], c.fx, c.fy, c.lim_x, c.lim_y,
           c.near_plane, c.far_plane, J);
  cov3d(q + g * 4, s + g * 3, sig);
  cov2d(J, Wm, sig, JW, cv);
  cov_out[g * 4 + 0] = cv[0][0];
  cov_out[g * 4 + 1] = cv[0][1];
  cov_out[g * 4 + 2] = cv[1][0];
  cov_out[g * 4 + 3] = cv[1][1];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      J_out[g * 6 + i * 3 + j] = J[i][j];
      JW_out[g * 6 + i * 3 + j] = JW[i][j];
    }
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      sig_out[g * 9 + i * 3 + j] = sig[i][j];
      W_out[g * 9 + i * 3 + j] = Wm[i][j];
    }
}

// compute_cov2d_backward (backward.cu:363-450): the chain on the saved
// J, Sigma, W, JW as passed in; grad_cam from the Jacobian chain only.
__global__ __launch_bounds__(256) void k_cov2d_bwd(
    const float* __restrict__ grad, const float* __restrict__ cam, const float* __restrict__ q,
    const float* __restrict__ s, const float* __restrict__ Jin, const float* __restrict__ sigin,
    const float* __restrict__ Win, const float* __restrict__ JWin, int64_t n, Cam c,
    float* __restrict__ gcam, float* __restrict__ gq, float* __restrict__ gs) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n) return;
  const float G2[2][2] = {{grad[g * 4 + 0], grad[g * 4 + 1]}, {grad[g * 4 + 2], grad[g * 4 + 3]}};
  float J[2][3], sig[3][3], Wm[3][3], JW[2][3], dSig[3][3], dJ[2][3], gj[3], dq[4], ds[3];
  load23(Jin + g * 6, J);
  load33(sigin + g * 9, sig);
  load33(Win + g * 9, Wm);
  load23(JWin + g * 6, JW);
  cov2d_chain_bwd(G2, J, Wm, sig, JW, dSig, dJ);
  jacobian_bwd(cam[g * 3 + 0], cam[g * 3 + 1], cam[g * 3 + 2], c.fx, c.fy, c.lim_x, c.lim_y,
               c.near_plane, c.far_plane, dJ, gj);
  cov3d_bwd(dSig, q + g * 4, s + g * 3, dq, ds);
#pragma unroll
  for (int i = 0; i < 3; ++i) gcam[g * 3 + i] = gj[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) gq[g * 4 + i] = dq[i];
#pragma unroll
  for (int i = 0; i < 3; ++i) gs[g * 3 + i] = ds[i];
}

// compute_means2d_kernel (forward.cu:297-330): clipped -> (1e6, 1e6).
__global__ __launch_bounds__(256) void k_means2d_fwd(const float* __restrict__ cam, int64_t n,
                                                     Cam c, float* __restrict__ out) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n) return;
  const float tx = cam[g * 3 + 0], ty = cam[g * 3 + 1], tz = cam[g * 3 + 2];
  float mx = 1e6f, my = 1e6f;
  if (!(tz <= c.near_plane || tz >= c.far_plane)) {
    const float inv_z = 1.0f / tz;
    const float px_div = -tx * inv_z;
    const float py_div = -ty * inv_z;
    mx = c.fx * px_div + c.px;
    my = c.fy * py_div + c.py;
  }
  out[g * 2 + 0] = mx;
  out[g * 2 + 1] = my;
}

__global__ __launch_bounds__(256) void k_means2d_bwd(const float* __restrict__ grad,
                                                     const float* __restrict__ cam, int64_t n,
                                                     Cam c, float* __restrict__ gcam) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n) return;
  float gm[3];
  means2d_bwd(cam[g * 3 + 0], cam[g * 3 + 1], cam[g * 3 + 2], c.fx, c.fy, c.near_plane,
              c.far_plane, grad[g * 2 + 0], grad[g * 2 + 1], gm);
#pragma unroll
  for (int i = 0; i < 3; ++i) gcam[g * 3 + i] = gm[i];
}

// invert_cov2d_kernel (forward.cu:333-356).
__global__ __launch_bounds__(256) void k_invert_fwd(const float* __restrict__ cov, int64_t n,
                                                    float* __restrict__ out) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n) return;
  const float a = cov[g * 4 + 0], b = cov[g * 4 + 1], c = cov[g * 4 + 2], d = cov[g * 4 + 3];
  const float det = a * d - b * c;
  const float inv_det = 1.0f / det;
  out[g * 4 + 0] = d * inv_det;
  out[g * 4 + 1] = -b * inv_det;
  out[g * 4 + 2] = -c * inv_det;
  out[g * 4 + 3] = a * inv_det;
}

// invert_cov2d_backward_kernel (backward.cu:500-543):
// grad = -(A^-1 (G A^-1)).
__global__ __launch_bounds__(256) void k_invert_bwd(const float* __restrict__ grad,
                                                    const float* __restrict__ cov, int64_t n,
                                                    float* __restrict__ out) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n) return;
  const float a = cov[g * 4 + 0], b = cov[g * 4 + 1], c = cov[g * 4 + 2], d = cov[g * 4 + 3];
  const float det = a * d - b * c;
  const float inv_det = 1.0f / det;
  const float ia = d * inv_det, ib = -b * inv_det, ic = -c * inv_det, id = a * inv_det;
  const float ga = grad[g * 4 + 0], gb = grad[g * 4 + 1], gc = grad[g * 4 + 2],
              gd = grad[g * 4 + 3];
  const float ta = ga * ia + gb * ic;
  const float tb = ga * ib + gb * id;
  const float tc = gc * ia + gd * ic;
  const float td = gc * ib + gd * id;
  out[g * 4 + 0] = -(ia * ta + ib * tc);
  out[g * 4 + 1] = -(ia * tb + ib * td);
  out[g * 4 + 2] = -(ic * ta + id * tc);
  out[g * 4 + 3] = -(ic * tb + id * td);
}

int check_n(int64_t n, const char* what) {
  if (n < 0 || n > (static_cast<int64_t>(1) << 40)) {
    set_error("%s: bad count %lld", what, static_cast<long long>(n));
    return HRF_ERR_INVALID;
  }
  return HRF_OK;
}

bool any_null(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (!p) return true;
  return false;
}

#define HRF_GEOM_LAUNCH(kernel, n, stream, ...)                                           \
  do {                                                                                    \
    if ((n) > 0) {                                                                        \
      hipLaunchKernelGGL(kernel, dim3(blocks_for((n), 256)), dim3(256), 0,                \
                         static_cast<hipStream_t>(stream), __VA_ARGS__);                  \
      HRF_LAUNCH_CHECK();                                                                 \
    }                                                                                     \
  } while (0)

#define HRF_GEOM_ARGS(name, n, ...)                                 \
  do {                                                              \
    HRF_TRY(check_n((n), name));                                    \
    if ((n) > 0 && any_null({__VA_ARGS__})) {                       \
      set_error("%s: null pointer", name);                          \
      return HRF_ERR_INVALID;                                       \
    }                                                               \
  } while (0)

}  // namespace
}  // namespace hrf

using namespace hrf;

extern "C" {

int hrf_cov3d_forward(const float* quats, const float* scales, int64_t n, float* cov3d,
                      void* stream) {
  HRF_GEOM_ARGS("cov3d_forward", n, quats, scales, cov3d);
  HRF_GEOM_LAUNCH(k_cov3d_fwd, n, stream, quats, scales, n, cov3d);
  return HRF_OK;
}

int hrf_cov3d_backward(const float* grad_cov3d, const float* quats, const float* scales,
                       int64_t n, float* grad_quats, float* grad_scales, void* stream) {
  HRF_GEOM_ARGS("cov3d_backward", n, grad_cov3d, quats, scales, grad_quats, grad_scales);
  HRF_GEOM_LAUNCH(k_cov3d_bwd, n, stream, grad_cov3d, quats, scales, n, grad_quats,
                  grad_scales);
  return HRF_OK;
}

int hrf_jacobian_forward(const float* cam_means, int64_t n, float fx, float fy, int32_t width,
                         int32_t height, float near_plane, float far_plane, float* jacobian,
                         void* stream) {
  HRF_GEOM_ARGS("jacobian_forward", n, cam_means, jacobian);
  const Cam c = make_cam(fx, fy, 0.f, 0.f, width, height, near_plane, far_plane);
  HRF_GEOM_LAUNCH(k_jacobian_fwd, n, stream, cam_means, n, c, jacobian);
  return HRF_OK;
}

int hrf_jacobian_backward(const float* grad_jacobian, const float* cam_means, int64_t n,
                          float fx, float fy, int32_t width, int32_t height, float near_plane,
                          float far_plane, float* grad_cam, void* stream) {
  HRF_GEOM_ARGS("jacobian_backward", n, grad_jacobian, cam_means, grad_cam);
  const Cam c = make_cam(fx, fy, 0.f, 0.f, width, height, near_plane, far_plane);
  HRF_GEOM_LAUNCH(k_jacobian_bwd, n, stream, grad_jacobian, cam_means, n, c, grad_cam);
  return HRF_OK;
}

int hrf_cov2d_forward(const float* cam_means, const float* quats, const float* scales,
                      const float* view_matrix, int64_t n, float fx, float fy, int32_t width,
                      int32_t height, float near_plane, float far_plane, float* cov2d,
                      float* jacobian, float* cov3d, float* view_rep, float* jw, void* stream) {
  HRF_GEOM_ARGS("cov2d_forward", n, cam_means, quats, scales, view_matrix, cov2d, jacobian,
                cov3d, view_rep, jw);
  const Cam c = make_cam(fx, fy, 0.f, 0.f, width, height, near_plane, far_plane);
  HRF_GEOM_LAUNCH(k_cov2d_fwd, n, stream, cam_means, quats, scales, view_matrix, n, c, cov2d,
                  jacobian, cov3d, view_rep, jw);
  return HRF_OK;
}

int hrf_cov2d_backward(const float* grad_cov2d, const float* cam_means, const float* quats,
                       const float* scales, const float* view_matrix, const float* jacobian,
                       const float* cov3d, const float* view_rep, const float* jw, int64_t n,
                       float fx, float fy, int32_t width, int32_t height, float near_plane,
                       float far_plane, float* grad_cam, float* grad_quats, float* grad_scales,
                       void* stream) {
  (void)view_matrix;  // the reference uses the repeated W it saved, not this
  HRF_GEOM_ARGS("cov2d_backward", n, grad_cov2d, cam_means, quats, scales, jacobian, cov3d,
                view_rep, jw, grad_cam, grad_quats, grad_scales);
  const Cam c = make_cam(fx, fy, 0.f, 0.f, width, height, near_plane, far_plane);
  HRF_GEOM_LAUNCH(k_cov2d_bwd, n, stream, grad_cov2d, cam_means, quats, scales, jacobian, cov3d,
                  view_rep, jw, n, c, grad_cam, grad_quats, grad_scales);
  return HRF_OK;
}

int hrf_means2d_forward(const float* cam_means, int64_t n, float fx, float fy, float px,
                        float py, float near_plane, float far_plane, float* means2d,
                        void* stream) {
  HRF_GEOM_ARGS("means2d_forward", n, cam_means, means2d);
  const Cam c = make_cam(fx, fy, px, py, 1, 1, near_plane, far_plane);
  HRF_GEOM_LAUNCH(k_means2d_fwd, n, stream, cam_means, n, c, means2d);
  return HRF_OK;
}

int hrf_means2d_backward(const float* grad_means2d, const float* cam_means, int64_t n, float fx,
                         float fy, float px, float py, float near_plane, float far_plane,
                         float* grad_cam, void* stream) {
  HRF_GEOM_ARGS("means2d_backward", n, grad_means2d, cam_means, grad_cam);
  const Cam c = make_cam(fx, fy, px, py, 1, 1, near_plane, far_plane);
  HRF_GEOM_LAUNCH(k_means2d_bwd, n, stream, grad_means2d, cam_means, n, c, grad_cam);
  return HRF_OK;
}

int hrf_invert_cov2d_forward(const float* cov2d, int64_t n, float* cov2d_inverse, void* stream) {
  HRF_GEOM_ARGS("invert_cov2d_forward", n, cov2d, cov2d_inverse);
  HRF_GEOM_LAUNCH(k_invert_fwd, n, stream, cov2d, n, cov2d_inverse);
  return HRF_OK;
}

int hrf_invert_cov2d_backward(const float* grad_inverse, const float* cov2d, int64_t n,
                              float* grad_cov2d, void* stream) {
  HRF_GEOM_ARGS("invert_cov2d_backward", n, grad_inverse, cov2d, grad_cov2d);
  HRF_GEOM_LAUNCH(k_invert_bwd, n, stream, grad_inverse, cov2d, n, grad_cov2d);
  return HRF_OK;
}

}  // extern "C"
