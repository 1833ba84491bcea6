// ssim.hip — the fused SSIM map and its image gradient (the `fast_ssim`
// name of the reference's cov3d_cuda module: python_import.py:43-58,449-454,
// kernels in cuda_prop/cov3d_cuda/conv.cu:935-1197).
//
// SSIM of two images x, y per channel with an 11x11 Gaussian window
// (sigma 1.5, weights summing to 1) and zero padding outside the image:
//   mu_x = w * x, mu_y = w * y, s_xx = w * x^2 - mu_x^2, s_yy likewise,
//   s_xy = w * (x y) - mu_x mu_y,
//   map = ((2 mu_x mu_y + C1)(2 s_xy + C2)) / ((mu_x^2 + mu_y^2 + C1)(s_xx + s_yy + C2)).
// The gradient is taken with respect to x only (as the reference): with
// A..D the four factors above and g the upstream gradient of the map,
//   a = g dmap/dmu_x, b = g dmap/d(w*x^2), c = g dmap/d(w*xy),
//   dL/dx = w * a + 2 x (w * b) + y (w * c)
// (the window is symmetric, so its adjoint is itself; zero padding makes the
// adjoint's padding zero as well).
//
// Work decomposition: one 256-thread block per 32x32 output tile of one
// channel.  The window is separable (the 2-D weights are products of the
// 1-D ones), so each block stages its input region with the halo in LDS,
// runs the 11-tap filter along the rows into LDS and then along the columns:
// 22 taps per statistic instead of 121.  The backward recomputes the
// statistics over the tile plus a 5-pixel halo (the support of the second
// window), forms a, b, c there in LDS and filters them in the same way, so
// it needs no workspace and reads x, y and g once per tile.
#include <cmath>

#include "hrf_internal.h"

namespace hrf {
namespace {

constexpr int kSsimTile = 32;
constexpr int kSsimR = 5;  // window radius (11 taps)
constexpr int kSsimThreads = 256;

struct SsimWeights {
  float w[2 * kSsimR + 1];
};

// 11-tap filter along a row of LDS.
__device__ __forceinline__ float tap_row(const float* row, const SsimWeights& g) {
  float v = 0.0f;
#pragma unroll
  for (int k = 0; k < 2 * kSsimR + 1; ++k) v = fmaf(g.w[k], row[k], v);
  return v;
}

// 11-tap filter down a column of LDS (stride ld).
__device__ __forceinline__ float tap_col(const float* col, int ld, const SsimWeights& g) {
  float v = 0.0f;
#pragma unroll
  for (int k = 0; k < 2 * kSsimR + 1; ++k) v = fmaf(g.w[k], col[k * ld], v);
  return v;
}

__device__ __forceinline__ float load_px(const float* img, int H, int W, int y, int x) {
  return (y >= 0 && y < H && x >= 0 && x < W) ? img[static_cast<int64_t>(y) * W + x] : 0.0f;
}

struct SsimStats {
  float mu1, mu2, s11, s22, s12;
};

// The SSIM factors in the reference's evaluation order
// (conv.cu:993-1001).
struct SsimTerms {
  float A, B, C, D;
};

__device__ __forceinline__ SsimTerms ssim_terms(const SsimStats& st, float C1, float C2) {
  SsimTerms t;
  const float mu1_sq = st.mu1 * st.mu1;
  const float mu2_sq = st.mu2 * st.mu2;
  const float mu1_mu2 = st.mu1 * st.mu2;
  t.C = 2.0f * mu1_mu2 + C1;
  t.D = 2.0f * st.s12 + C2;
  t.A = mu1_sq + mu2_sq + C1;
  t.B = st.s11 + st.s22 + C2;
  return t;
}

// Forward: region of (32 + 10)^2 inputs -> 32 x 32 outputs.
constexpr int kFwdIn = kSsimTile + 2 * kSsimR;  // 42
constexpr int kFwdLd = kFwdIn + 1;              // LDS row pitch (odd: no bank aliasing)

__global__ __launch_bounds__(kSsimThreads) void k_ssim_map(const float* __restrict__ img1,
                                                          const float* __restrict__ img2, int H,
                                                          int W, float C1, float C2,
                                                          SsimWeights g,
                                                          float* __restrict__ map) {
  __shared__ float s_x[kFwdIn * kFwdLd];
  __shared__ float s_y[kFwdIn * kFwdLd];
  // Row-filtered statistics: 5 x (42 rows x 32 columns).
  __shared__ float s_h[5][kFwdIn * kSsimTile];
  const int64_t plane = static_cast<int64_t>(blockIdx.z) * H * W;
  const float* x = img1 + plane;
  const float* y = img2 + plane;
  const int oy = blockIdx.y * kSsimTile, ox = blockIdx.x * kSsimTile;
  for (int i = threadIdx.x; i < kFwdIn * kFwdIn; i += kSsimThreads) {
    const int r = i / kFwdIn, c = i - r * kFwdIn;
    s_x[r * kFwdLd + c] = load_px(x, H, W, oy - kSsimR + r, ox - kSsimR + c);
    s_y[r * kFwdLd + c] = load_px(y, H, W, oy - kSsimR + r, ox - kSsimR + c);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kFwdIn * kSsimTile; i += kSsimThreads) {
    const int r = i / kSsimTile, c = i - r * kSsimTile;
    const float* px = s_x + r * kFwdLd + c;
    const float* py = s_y + r * kFwdLd + c;
    float m1 = 0.0f, m2 = 0.0f, e11 = 0.0f, e22 = 0.0f, e12 = 0.0f;
#pragma unroll
    for (int k = 0; k < 2 * kSsimR + 1; ++k) {
      const float a = px[k], b = py[k], w = g.w[k];
      m1 = fmaf(w, a, m1);
      m2 = fmaf(w, b, m2);
      e11 = fmaf(w, a * a, e11);
      e22 = fmaf(w, b * b, e22);
      e12 = fmaf(w, a * b, e12);
    }
    s_h[0][i] = m1;
    s_h[1][i] = m2;
    s_h[2][i] = e11;
    s_h[3][i] = e22;
    s_h[4][i] = e12;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kSsimTile * kSsimTile; i += kSsimThreads) {
    const int r = i / kSsimTile, c = i - r * kSsimTile;
    const int py = oy + r, px = ox + c;
    if (py >= H || px >= W) continue;
    const int o = r * kSsimTile + c;
    SsimStats st;
    st.mu1 = tap_col(s_h[0] + o, kSsimTile, g);
    st.mu2 = tap_col(s_h[1] + o, kSsimTile, g);
    st.s11 = tap_col(s_h[2] + o, kSsimTile, g) - st.mu1 * st.mu1;
    st.s22 = tap_col(s_h[3] + o, kSsimTile, g) - st.mu2 * st.mu2;
    st.s12 = tap_col(s_h[4] + o, kSsimTile, g) - st.mu1 * st.mu2;
    const SsimTerms t = ssim_terms(st, C1, C2);
    map[plane + static_cast<int64_t>(py) * W + px] = (t.C * t.D) / (t.A * t.B);
  }
}

// Backward: inputs over (32 + 20)^2, statistics and a, b, c over
// (32 + 10)^2, gradient over 32 x 32.
constexpr int kBwdIn = kSsimTile + 4 * kSsimR;  // 52
constexpr int kBwdLd = kBwdIn + 1;
constexpr int kBwdMid = kSsimTile + 2 * kSsimR;  // 42
constexpr int kBwdMidLd = kBwdMid + 1;

__global__ __launch_bounds__(kSsimThreads) void k_ssim_backward(
    const float* __restrict__ img1, const float* __restrict__ img2,
    const float* __restrict__ grad_map, int H, int W, float C1, float C2, SsimWeights g,
    float* __restrict__ grad_img1) {
  __shared__ float s_x[kBwdIn * kBwdLd];
  __shared__ float s_y[kBwdIn * kBwdLd];
  // Row-filtered statistics (5 x 52 rows x 42 columns); afterwards reused
  // for the row-filtered a, b, c (3 x 42 rows x 32 columns).
  __shared__ float s_h[5 * kBwdIn * kBwdMid];
  __shared__ float s_abc[3][kBwdMid * kBwdMidLd];
  const int64_t plane = static_cast<int64_t>(blockIdx.z) * H * W;
  const float* x = img1 + plane;
  const float* y = img2 + plane;
  const float* gm = grad_map + plane;
  const int oy = blockIdx.y * kSsimTile, ox = blockIdx.x * kSsimTile;
  const int y0 = oy - 2 * kSsimR, x0 = ox - 2 * kSsimR;  // input region origin
  for (int i = threadIdx.x; i < kBwdIn * kBwdIn; i += kSsimThreads) {
    const int r = i / kBwdIn, c = i - r * kBwdIn;
    s_x[r * kBwdLd + c] = load_px(x, H, W, y0 + r, x0 + c);
    s_y[r * kBwdLd + c] = load_px(y, H, W, y0 + r, x0 + c);
  }
  __syncthreads();
  constexpr int kHN = kBwdIn * kBwdMid;  // one statistic's row-filtered block
  for (int i = threadIdx.x; i < kHN; i += kSsimThreads) {
    const int r = i / kBwdMid, c = i - r * kBwdMid;
    const float* px = s_x + r * kBwdLd + c;
    const float* py = s_y + r * kBwdLd + c;
    float m1 = 0.0f, m2 = 0.0f, e11 = 0.0f, e22 = 0.0f, e12 = 0.0f;
#pragma unroll
    for (int k = 0; k < 2 * kSsimR + 1; ++k) {
      const float a = px[k], b = py[k], w = g.w[k];
      m1 = fmaf(w, a, m1);
      m2 = fmaf(w, b, m2);
      e11 = fmaf(w, a * a, e11);
      e22 = fmaf(w, b * b, e22);
      e12 = fmaf(w, a * b, e12);
    }
    s_h[0 * kHN + i] = m1;
    s_h[1 * kHN + i] = m2;
    s_h[2 * kHN + i] = e11;
    s_h[3 * kHN + i] = e22;
    s_h[4 * kHN + i] = e12;
  }
  __syncthreads();
  // Statistics at the 42 x 42 positions around the tile; a, b, c there
  // (zero outside the image, where the map has no gradient).
  for (int i = threadIdx.x; i < kBwdMid * kBwdMid; i += kSsimThreads) {
    const int r = i / kBwdMid, c = i - r * kBwdMid;
    const int py = oy - kSsimR + r, px = ox - kSsimR + c;
    float a = 0.0f, b = 0.0f, cc = 0.0f;
    if (py >= 0 && py < H && px >= 0 && px < W) {
      const int o = r * kBwdMid + c;
      SsimStats st;
      st.mu1 = tap_col(s_h + 0 * kHN + o, kBwdMid, g);
      st.mu2 = tap_col(s_h + 1 * kHN + o, kBwdMid, g);
      st.s11 = tap_col(s_h + 2 * kHN + o, kBwdMid, g) - st.mu1 * st.mu1;
      st.s22 = tap_col(s_h + 3 * kHN + o, kBwdMid, g) - st.mu2 * st.mu2;
      st.s12 = tap_col(s_h + 4 * kHN + o, kBwdMid, g) - st.mu1 * st.mu2;
      const SsimTerms t = ssim_terms(st, C1, C2);
      const float dm = gm[static_cast<int64_t>(py) * W + px];
      const float AB = t.A * t.B;
      // d map / d mu1 (the w*x^2 and w*xy statistics held fixed),
      // d map / d(w*x^2), d map / d(w*xy)  (conv.cu:1081-1088)
      a = dm * ((st.mu2 * 2.0f * t.D) / AB - (st.mu2 * 2.0f * t.C) / AB -
                (st.mu1 * 2.0f * t.C * t.D) / (t.A * t.A * t.B) +
                (st.mu1 * 2.0f * t.C * t.D) / (AB * t.B));
      b = dm * ((-t.C * t.D) / (AB * t.B));
      cc = dm * ((2.0f * t.C) / AB);
    }
    s_abc[0][r * kBwdMidLd + c] = a;
    s_abc[1][r * kBwdMidLd + c] = b;
    s_abc[2][r * kBwdMidLd + c] = cc;
  }
  __syncthreads();
  constexpr int kH2 = kBwdMid * kSsimTile;
  for (int i = threadIdx.x; i < kH2; i += kSsimThreads) {
    const int r = i / kSsimTile, c = i - r * kSsimTile;
#pragma unroll
    for (int q = 0; q < 3; ++q) s_h[q * kH2 + i] = tap_row(&s_abc[q][r * kBwdMidLd + c], g);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kSsimTile * kSsimTile; i += kSsimThreads) {
    const int r = i / kSsimTile, c = i - r * kSsimTile;
    const int py = oy + r, px = ox + c;
    if (py >= H || px >= W) continue;
    const int o = r * kSsimTile + c;
    const float wa = tap_col(s_h + 0 * kH2 + o, kSsimTile, g);
    const float wb = tap_col(s_h + 1 * kH2 + o, kSsimTile, g);
    const float wc = tap_col(s_h + 2 * kH2 + o, kSsimTile, g);
    const float xv = s_x[(r + 2 * kSsimR) * kBwdLd + c + 2 * kSsimR];
    const float yv = s_y[(r + 2 * kSsimR) * kBwdLd + c + 2 * kSsimR];
    grad_img1[plane + static_cast<int64_t>(py) * W + px] = wa + xv * (2.0f * wb) + yv * wc;
  }
}

// The 1-D window: exp(-(k-5)^2 / (2 sigma^2)), sigma = 1.5, normalised to
// sum 1 (in double, then rounded).
SsimWeights ssim_weights() {
  SsimWeights g;
  double w[2 * kSsimR + 1], sum = 0.0;
  for (int k = 0; k <= 2 * kSsimR; ++k) {
    const double d = static_cast<double>(k - kSsimR);
    w[k] = std::exp(-d * d / (2.0 * 1.5 * 1.5));
    sum += w[k];
  }
  for (int k = 0; k <= 2 * kSsimR; ++k) g.w[k] = static_cast<float>(w[k] / sum);
  return g;
}

int check_ssim(int C, int H, int W) {
  if (C < 1 || H < 1 || W < 1 || static_cast<int64_t>(C) > 65535 ||
      static_cast<int64_t>(C) * H * W > (int64_t(1) << 40)) {
    set_error("ssim: invalid image shape (%d, %d, %d)", C, H, W);
    return HRF_ERR_INVALID;
  }
  return HRF_OK;
}

dim3 ssim_grid(int C, int H, int W) {
  return dim3((W + kSsimTile - 1) / kSsimTile, (H + kSsimTile - 1) / kSsimTile, C);
}

}  // namespace
}  // namespace hrf

using namespace hrf;

extern "C" {

int hrf_ssim_map(const float* img1, const float* img2, int32_t channels, int32_t height,
                 int32_t width, float c1, float c2, float* ssim_map, void* stream) {
  HRF_TRY(check_ssim(channels, height, width));
  if (!img1 || !img2 || !ssim_map) {
    set_error("ssim: null pointer");
    return HRF_ERR_INVALID;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  HRF_STAGE("ssim", s);
  hipLaunchKernelGGL(k_ssim_map, ssim_grid(channels, height, width), dim3(kSsimThreads), 0, s,
                     img1, img2, height, width, c1, c2, ssim_weights(), ssim_map);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int hrf_ssim_backward(const float* img1, const float* img2, const float* grad_map,
                      int32_t channels, int32_t height, int32_t width, float c1, float c2,
                      float* grad_img1, void* stream) {
  HRF_TRY(check_ssim(channels, height, width));
  if (!img1 || !img2 || !grad_map || !grad_img1) {
    set_error("ssim: null pointer");
    return HRF_ERR_INVALID;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  HRF_STAGE("ssim", s);
  hipLaunchKernelGGL(k_ssim_backward, ssim_grid(channels, height, width), dim3(kSsimThreads), 0,
                     s, img1, img2, grad_map, height, width, c1, c2, ssim_weights(), grad_img1);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

}  // extern "C"
