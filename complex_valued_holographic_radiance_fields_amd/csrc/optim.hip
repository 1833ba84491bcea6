// optim.hip — the training step's optimizer side, fused: the global
// gradient-norm clip and the Adan update over every parameter tensor in one
// launch each.
//
// Reference: train.py:319-324 (torch.nn.utils.clip_grad_norm_(parameters,
// 1.0), then Adan.step()), utils/optimizer.py:288-466 (Adan, its defaults and
// state) and :538-589 (_multi_tensor_adan, the foreach path the reference
// runs).  The reference issues ~20 foreach kernels per step (each a full
// pass over all seven tensors) plus the norm; here the norm is one pass over
// the gradients (per-block partial sums, summed in a fixed order by one
// block that also forms the clip coefficient on the device), and the update
// one pass that reads param, grad and the four state tensors once and
// writes them once.  The clip coefficient is applied inside the update
// (and the scaled gradient written back), so the separate rescaling pass of
// clip_grad_norm_ is optional.
#include <cmath>
#include <mutex>
#include <vector>

#include "hrf_internal.h"

namespace hrf {

// Scratch of hrf_grad_norm_static: the per-chunk partial sums of squares,
// one float per 2048 gradient elements, in a file-scope device array instead
// of a caller workspace (each GPU the library runs on holds its own copy,
// 256 KiB, until the process ends).  In host code this name is only a
// stand-in for the symbol: the device address comes from
// hipGetSymbolAddress, once per device (static_norm_scratch below).
constexpr int kStaticNormPartials = 65536;
static __device__ __align__(256) float scratch[kStaticNormPartials];

namespace {

constexpr int kOptThreads = 256;
constexpr int kOptItems = 8;                            // elements per thread
constexpr int kOptChunk = kOptThreads * kOptItems;       // elements per block
constexpr int kMaxOptTensors = 8;                        // per launch
constexpr int kNormFinalThreads = 1024;

// Per-launch table: tensor t owns blocks [first[t], first[t + 1]).
struct AdanTable {
  float* p[kMaxOptTensors];
  float* g[kMaxOptTensors];
  float* m[kMaxOptTensors];
  float* n[kMaxOptTensors];
  float* d[kMaxOptTensors];
  float* q[kMaxOptTensors];  // neg_pre_grad
  int64_t numel[kMaxOptTensors];
  // Host-formed scalars (double arithmetic, then rounded, as the reference's
  // Python floats reach its kernels): step_size = lr / bc1, step_size_diff =
  // lr * beta2 / bc2, sqrt(bc3), 1 + lr * weight_decay, 1 - lr * weight_decay.
  float step_size[kMaxOptTensors];
  float step_size_diff[kMaxOptTensors];
  float bc3_sqrt[kMaxOptTensors];
  float wd_div[kMaxOptTensors];
  float wd_mul[kMaxOptTensors];
  int init_npg[kMaxOptTensors];  // the group's first step: neg_pre_grad = -grad
  int vec[kMaxOptTensors];       // all six pointers 16-byte aligned
  int first[kMaxOptTensors + 1];
  int count;
};

struct AdanScalars {
  float beta1, beta2, beta3, one_m_b1, one_m_b2, one_m_b3, eps, clip;
  int no_prox, wd;  // wd: weight decay nonzero
};

struct GradTable {
  const float* g[kMaxOptTensors];
  int64_t numel[kMaxOptTensors];
  int first[kMaxOptTensors + 1];
  int count;
};

template <typename Table>
__device__ __forceinline__ int tensor_of(const Table& t, int b) {
  int k = 0;
#pragma unroll
  for (int i = 1; i < kMaxOptTensors; ++i) k += (i < t.count && b >= t.first[i]) ? 1 : 0;
  return k;
}

// One element of _multi_tensor_adan (optimizer.py:556-589), op by op in
// float32 (the library is built without contraction).
__device__ __forceinline__ void adan_elem(float& p, float& g, float& m, float& n, float& d,
                                          float& q, float scale, const AdanScalars& s,
                                          float step_size, float step_size_diff,
                                          float bc3_sqrt, float wd_div, float wd_mul,
                                          bool init) {
  g = g * scale;                         // clip_grad_norm_ coefficient (1 if none)
  g = g * s.clip;                        // _foreach_mul_(grads, clip_global_grad_norm)
  if (init) q = -g;                      // neg_pre_grad = grad * -clip (step 1)
  q = q + g;                             // _foreach_add_(neg_pre_grads, grads)
  m = m * s.beta1;
  m = m + s.one_m_b1 * g;                // m_t
  d = d * s.beta2;
  d = d + s.one_m_b2 * q;                // diff_t
  q = q * s.beta2;
  q = q + g;
  n = n * s.beta3;
  n = n + s.one_m_b3 * q * q;            // n_t (addcmul: value * t1 * t2)
  float denom = sqrtf(n);
  denom = denom / bc3_sqrt;
  denom = denom + s.eps;
  if (s.no_prox) {
    p = p * wd_mul;
    p = p + (-step_size) * (m / denom);
    p = p + (-step_size_diff) * (d / denom);
  } else {
    p = p + (-step_size) * (m / denom);
    p = p + (-step_size_diff) * (d / denom);
    if (s.wd) p = p / wd_div;
  }
  q = -g;                                // zero_() then add_(grads, alpha=-1)
}

__global__ __launch_bounds__(kOptThreads) void k_adan(AdanTable t, AdanScalars s,
                                                      const float* __restrict__ grad_scale) {
  const int k = tensor_of(t, blockIdx.x);
  const int64_t n_el = t.numel[k];
  const int64_t base = static_cast<int64_t>(blockIdx.x - t.first[k]) * kOptChunk;
  const float scale = grad_scale ? *grad_scale : 1.0f;
  const float ss = t.step_size[k], ssd = t.step_size_diff[k], b3 = t.bc3_sqrt[k];
  const float wdd = t.wd_div[k], wdm = t.wd_mul[k];
  const bool init = t.init_npg[k] != 0;
  float* __restrict__ P = t.p[k];
  float* __restrict__ G = t.g[k];
  float* __restrict__ M = t.m[k];
  float* __restrict__ N = t.n[k];
  float* __restrict__ D = t.d[k];
  float* __restrict__ Q = t.q[k];
  if (t.vec[k]) {
    // Two float4 groups per thread: kOptItems / 4 = 2.
#pragma unroll
    for (int u = 0; u < kOptItems / 4; ++u) {
      const int64_t i = base + 4 * (static_cast<int64_t>(u) * kOptThreads + threadIdx.x);
      if (i + 3 < n_el) {
        float4 p4 = *reinterpret_cast<float4*>(P + i), g4 = *reinterpret_cast<float4*>(G + i);
        float4 m4 = *reinterpret_cast<float4*>(M + i), n4 = *reinterpret_cast<float4*>(N + i);
        float4 d4 = *reinterpret_cast<float4*>(D + i), q4 = *reinterpret_cast<float4*>(Q + i);
        adan_elem(p4.x, g4.x, m4.x, n4.x, d4.x, q4.x, scale, s, ss, ssd, b3, wdd, wdm, init);
        adan_elem(p4.y, g4.y, m4.y, n4.y, d4.y, q4.y, scale, s, ss, ssd, b3, wdd, wdm, init);
        adan_elem(p4.z, g4.z, m4.z, n4.z, d4.z, q4.z, scale, s, ss, ssd, b3, wdd, wdm, init);
        adan_elem(p4.w, g4.w, m4.w, n4.w, d4.w, q4.w, scale, s, ss, ssd, b3, wdd, wdm, init);
        *reinterpret_cast<float4*>(P + i) = p4;
        *reinterpret_cast<float4*>(G + i) = g4;
        *reinterpret_cast<float4*>(M + i) = m4;
        *reinterpret_cast<float4*>(N + i) = n4;
        *reinterpret_cast<float4*>(D + i) = d4;
        *reinterpret_cast<float4*>(Q + i) = q4;
      } else {
        for (int64_t j = i; j < n_el && j < i + 4; ++j)
          adan_elem(P[j], G[j], M[j], N[j], D[j], Q[j], scale, s, ss, ssd, b3, wdd, wdm, init);
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < kOptItems; ++u) {
      const int64_t j = base + static_cast<int64_t>(u) * kOptThreads + threadIdx.x;
      if (j < n_el)
        adan_elem(P[j], G[j], M[j], N[j], D[j], Q[j], scale, s, ss, ssd, b3, wdd, wdm, init);
    }
  }
}

// Sum of squares of one chunk per block -> partial[block] (fixed order).
__global__ __launch_bounds__(kOptThreads) void k_sumsq(GradTable t, float* __restrict__ partial,
                                                       int partial_off) {
  __shared__ float s_w[kOptThreads / 64];
  const int k = tensor_of(t, blockIdx.x);
  const int64_t n_el = t.numel[k];
  const int64_t base = static_cast<int64_t>(blockIdx.x - t.first[k]) * kOptChunk;
  const float* __restrict__ G = t.g[k];
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kOptItems; ++u) {
    const int64_t j = base + static_cast<int64_t>(u) * kOptThreads + threadIdx.x;
    const float v = j < n_el ? G[j] : 0.0f;
    acc = fmaf(v, v, acc);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = 0.0f;
#pragma unroll
    for (int w = 0; w < kOptThreads / 64; ++w) b += s_w[w];
    partial[partial_off + blockIdx.x] = b;
  }
}

// One block: total = sqrt(sum of the partials), coef = clamp(max_norm /
// (total + 1e-6), max = 1) as clip_grad_norm_ forms it (NaN propagates).
__global__ __launch_bounds__(kNormFinalThreads) void k_norm_final(const float* __restrict__ partial,
                                                                  int np, float max_norm,
                                                                  float* __restrict__ total_out,
                                                                  float* __restrict__ coef_out) {
  __shared__ float s_w[kNormFinalThreads / 64];
  float acc = 0.0f;
  for (int i = threadIdx.x; i < np; i += kNormFinalThreads) acc += partial[i];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = 0.0f;
    for (int w = 0; w < kNormFinalThreads / 64; ++w) b += s_w[w];
    const float total = sqrtf(b);
    float coef = max_norm / (total + 1e-6f);
    coef = coef > 1.0f ? 1.0f : coef;
    if (total_out) *total_out = total;
    if (coef_out) *coef_out = coef;
  }
}

__global__ __launch_bounds__(kOptThreads) void k_scale(GradTable t, const float* __restrict__ coef) {
  const int k = tensor_of(t, blockIdx.x);
  const int64_t n_el = t.numel[k];
  const int64_t base = static_cast<int64_t>(blockIdx.x - t.first[k]) * kOptChunk;
  float* __restrict__ G = const_cast<float*>(t.g[k]);
  const float c = *coef;
#pragma unroll
  for (int u = 0; u < kOptItems; ++u) {
    const int64_t j = base + static_cast<int64_t>(u) * kOptThreads + threadIdx.x;
    if (j < n_el) G[j] = G[j] * c;
  }
}

int64_t chunks_of(int64_t numel) { return (numel + kOptChunk - 1) / kOptChunk; }

int64_t total_elems(const int64_t* numels, int nt) {
  int64_t c = 0;
  for (int i = 0; i < nt; ++i) c += numels[i];
  return c;
}

// Device address of `scratch` on the current device, looked up once per
// device (each device holds its own copy of the array at its own address).
// Host code passes this address, never the array's name, to the kernels.
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxScratchDevices] = {};

int static_norm_scratch(float** out) {
  int dev = 0;
  HRF_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxScratchDevices) {
    set_error("grad norm (static scratch): device %d out of range", dev);
    return HRF_ERR_INVALID;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    HRF_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) {
      set_error("grad norm (static scratch): no device address for the scratch array");
      return HRF_ERR_HIP;
    }
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return HRF_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Blocks of all tensors, the norm's partial-sum count.
int64_t total_chunks(const int64_t* numels, int nt) {
  int64_t c = 0;
  for (int i = 0; i < nt; ++i) c += chunks_of(numels[i]);
  return c;
}

// traced: open the "grad_norm" stage timer (hipEvents, taken from a pool
// that grows on demand, when stage tracing is on).  The allocation-free
// entry point passes false.
int launch_grad_norm(const float* const* grads, const int64_t* numels, int num_tensors,
                     float max_norm, float* total_norm, float* clip_coef, float* partial,
                     hipStream_t s, bool traced = true);

int check_grad_list(const float* const* grads, const int64_t* numels, int nt) {
  if (nt < 0 || (nt > 0 && (!grads || !numels))) {
    set_error("optimizer: invalid tensor list");
    return HRF_ERR_INVALID;
  }
  for (int i = 0; i < nt; ++i) {
    if (numels[i] < 0 || (numels[i] > 0 && !grads[i])) {
      set_error("optimizer: tensor %d has a null pointer or negative size", i);
      return HRF_ERR_INVALID;
    }
    if (chunks_of(numels[i]) > 0x3FFFFFFF) {
      set_error("optimizer: tensor %d too large", i);
      return HRF_ERR_INVALID;
    }
  }
  return HRF_OK;
}

// Launches `kernel` over the tensors in groups of kMaxOptTensors (skipping
// empty ones); `fill(table, slot, tensor index)` sets a slot.
template <typename Table, typename Fill, typename Launch>
int for_tensor_groups(int nt, const int64_t* numels, Fill fill, Launch launch) {
  int i = 0;
  int64_t block_off = 0;
  while (i < nt) {
    Table t{};
    int blocks = 0;
    t.first[0] = 0;
    while (i < nt && t.count < kMaxOptTensors) {
      if (numels[i] > 0) {
        fill(t, t.count, i);
        t.numel[t.count] = numels[i];
        blocks += static_cast<int>(chunks_of(numels[i]));
        t.first[t.count + 1] = blocks;
        ++t.count;
      }
      ++i;
    }
    for (int k = t.count + 1; k <= kMaxOptTensors; ++k) t.first[k] = blocks;
    if (blocks > 0) {
      HRF_TRY(launch(t, blocks, block_off));
      block_off += blocks;
    }
  }
  return HRF_OK;
}


// Sparse Adam over the visible rows (spadam.cu:8-36, the `adamUpdate` behind
// python_import.py:457-460): param, exp_avg, exp_avg_sq are (B, N, D), grad
// (B, V, D) holds the gradients of the V visible rows, visible (V) their row
// indices.  No bias correction, as the reference.  One thread per element of
// (B, V, D) in row-major order, so a row's D elements are contiguous in both
// the gathered gradient and the parameter tensors.  Rows outside [0, N) are
// skipped (the reference writes out of bounds); duplicate rows race, as in
// the reference.
__global__ __launch_bounds__(kOptThreads) void k_sparse_adam(
    float* __restrict__ param, const float* __restrict__ grad, float* __restrict__ exp_avg,
    float* __restrict__ exp_avg_sq, const int64_t* __restrict__ visible, int64_t B, int64_t N,
    int64_t V, int64_t D, float lr, float b1, float b2, float eps) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kOptThreads + threadIdx.x;
  const int64_t total = B * V * D;
  if (i >= total) return;
  const int64_t d = i % D;
  const int64_t bv = i / D;
  const int64_t v = bv % V, b = bv / V;
  const int64_t row = visible[v];
  if (row < 0 || row >= N) return;
  const int64_t at = (b * N + row) * D + d;
  const float gr = grad[i];
  float m = exp_avg[at];
  float s2 = exp_avg_sq[at];
  m = b1 * m + (1.0f - b1) * gr;
  s2 = b2 * s2 + (1.0f - b2) * gr * gr;
  const float step = -lr * m / (sqrtf(s2) + eps);
  param[at] += step;
  exp_avg[at] = m;
  exp_avg_sq[at] = s2;
}
}  // namespace
}  // namespace hrf

using namespace hrf;

extern "C" {

size_t hrf_grad_norm_workspace_size(const int64_t* numels, int32_t num_tensors) {
  if (num_tensors < 0 || (num_tensors > 0 && !numels)) return 0;
  return static_cast<size_t>(total_chunks(numels, num_tensors) + 1) * sizeof(float);
}

int hrf_grad_norm(const float* const* grads, const int64_t* numels, int32_t num_tensors,
                  float max_norm, float* total_norm, float* clip_coef, void* ws,
                  size_t ws_bytes, void* stream) {
  HRF_TRY(check_grad_list(grads, numels, num_tensors));
  if (!total_norm && !clip_coef) {
    set_error("grad norm: no output");
    return HRF_ERR_INVALID;
  }
  const size_t need = hrf_grad_norm_workspace_size(numels, num_tensors);
  if (!ws || ws_bytes < need) {
    set_error("grad norm workspace too small: %zu bytes given, %zu needed", ws_bytes, need);
    return HRF_ERR_WORKSPACE;
  }
  return launch_grad_norm(grads, numels, num_tensors, max_norm, total_norm, clip_coef,
                          static_cast<float*>(ws), static_cast<hipStream_t>(stream));
}

int hrf_grad_norm_static(const float* const* grads, const int64_t* numels, int32_t num_tensors,
                         float max_norm, float* total_norm, float* clip_coef, void* stream) {
  HRF_TRY(check_grad_list(grads, numels, num_tensors));
  if (!total_norm && !clip_coef) {
    set_error("grad norm: no output");
    return HRF_ERR_INVALID;
  }
  const int64_t chunks = total_chunks(numels, num_tensors);
  if (chunks > kStaticNormPartials) {
    set_error("grad norm (static scratch): %lld gradient elements need %lld partial sums; the "
              "static scratch holds %d (at most %lld elements); use hrf_grad_norm with a "
              "workspace",
              static_cast<long long>(total_elems(numels, num_tensors)),
              static_cast<long long>(chunks), kStaticNormPartials,
              static_cast<long long>(kStaticNormPartials) * kOptChunk);
    return HRF_ERR_WORKSPACE;
  }
  float* partial = nullptr;
  HRF_TRY(static_norm_scratch(&partial));
  return launch_grad_norm(grads, numels, num_tensors, max_norm, total_norm, clip_coef, partial,
                          static_cast<hipStream_t>(stream), /*traced=*/false);
}

}  // extern "C"

namespace hrf {
namespace {

int launch_grad_norm(const float* const* grads, const int64_t* numels, int num_tensors,
                     float max_norm, float* total_norm, float* clip_coef, float* partial,
                     hipStream_t s, bool traced) {
  if (traced) {
    HRF_STAGE("grad_norm", s);
    return launch_grad_norm(grads, numels, num_tensors, max_norm, total_norm, clip_coef, partial,
                            s, false);
  }
  HRF_TRY(for_tensor_groups<GradTable>(
      num_tensors, numels, [&](GradTable& t, int slot, int i) { t.g[slot] = grads[i]; },
      [&](const GradTable& t, int blocks, int64_t off) -> int {
        hipLaunchKernelGGL(k_sumsq, dim3(blocks), dim3(kOptThreads), 0, s, t, partial,
                           static_cast<int>(off));
        HRF_LAUNCH_CHECK();
        return HRF_OK;
      }));
  const int np = static_cast<int>(total_chunks(numels, num_tensors));
  hipLaunchKernelGGL(k_norm_final, dim3(1), dim3(kNormFinalThreads), 0, s, partial, np, max_norm,
                     total_norm, clip_coef);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

}  // namespace
}  // namespace hrf

extern "C" {

int hrf_scale_grads(float* const* grads, const int64_t* numels, int32_t num_tensors,
                    const float* coef, void* stream) {
  HRF_TRY(check_grad_list(const_cast<const float* const*>(grads), numels, num_tensors));
  if (!coef) {
    set_error("scale grads: null coefficient");
    return HRF_ERR_INVALID;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  HRF_STAGE("grad_scale", s);
  return for_tensor_groups<GradTable>(
      num_tensors, numels, [&](GradTable& t, int slot, int i) { t.g[slot] = grads[i]; },
      [&](const GradTable& t, int blocks, int64_t) -> int {
        hipLaunchKernelGGL(k_scale, dim3(blocks), dim3(kOptThreads), 0, s, t, coef);
        HRF_LAUNCH_CHECK();
        return HRF_OK;
      });
}

int hrf_adan_step(const hrf_adan_tensor* tensors, int32_t num_tensors,
                  const hrf_adan_config* cfg, const float* grad_scale, void* stream) {
  if (num_tensors < 0 || (num_tensors > 0 && !tensors) || !cfg) {
    set_error("adan: invalid arguments");
    return HRF_ERR_INVALID;
  }
  const double b1 = cfg->beta1, b2 = cfg->beta2, b3 = cfg->beta3;
  if (!(b1 >= 0.0 && b1 < 1.0) || !(b2 >= 0.0 && b2 < 1.0) || !(b3 >= 0.0 && b3 < 1.0) ||
      !(cfg->eps >= 0.0)) {
    set_error("adan: invalid betas or eps");
    return HRF_ERR_INVALID;
  }
  std::vector<int64_t> numels(static_cast<size_t>(num_tensors));
  for (int i = 0; i < num_tensors; ++i) {
    const hrf_adan_tensor& t = tensors[i];
    numels[i] = t.numel;
    if (t.numel < 0 || (t.numel > 0 && (!t.param || !t.grad || !t.exp_avg || !t.exp_avg_sq ||
                                        !t.exp_avg_diff || !t.neg_pre_grad))) {
      set_error("adan: tensor %d has a null pointer or negative size", i);
      return HRF_ERR_INVALID;
    }
    if (t.numel > 0 && (t.step < 1 || !(t.lr >= 0.0))) {
      set_error("adan: tensor %d needs step >= 1 and lr >= 0", i);
      return HRF_ERR_INVALID;
    }
    if (chunks_of(t.numel) > 0x3FFFFFFF) {
      set_error("adan: tensor %d too large", i);
      return HRF_ERR_INVALID;
    }
  }
  AdanScalars sc;
  sc.beta1 = static_cast<float>(b1);
  sc.beta2 = static_cast<float>(b2);
  sc.beta3 = static_cast<float>(b3);
  sc.one_m_b1 = static_cast<float>(1.0 - b1);
  sc.one_m_b2 = static_cast<float>(1.0 - b2);
  sc.one_m_b3 = static_cast<float>(1.0 - b3);
  sc.eps = static_cast<float>(cfg->eps);
  sc.clip = static_cast<float>(cfg->clip_global_grad_norm);
  sc.no_prox = cfg->no_prox != 0;
  sc.wd = cfg->weight_decay != 0.0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  HRF_STAGE("adan", s);
  return for_tensor_groups<AdanTable>(
      num_tensors, numels.data(),
      [&](AdanTable& t, int slot, int i) {
        const hrf_adan_tensor& a = tensors[i];
        t.p[slot] = a.param;
        t.g[slot] = a.grad;
        t.m[slot] = a.exp_avg;
        t.n[slot] = a.exp_avg_sq;
        t.d[slot] = a.exp_avg_diff;
        t.q[slot] = a.neg_pre_grad;
        const double step = static_cast<double>(a.step);
        const double bc1 = 1.0 - std::pow(b1, step), bc2 = 1.0 - std::pow(b2, step);
        const double bc3 = 1.0 - std::pow(b3, step);
        const double lr = a.lr;
        t.step_size[slot] = static_cast<float>(lr / bc1);
        t.step_size_diff[slot] = static_cast<float>(lr * b2 / bc2);
        t.bc3_sqrt[slot] = static_cast<float>(std::sqrt(bc3));
        t.wd_div[slot] = static_cast<float>(1.0 + lr * cfg->weight_decay);
        t.wd_mul[slot] = static_cast<float>(1.0 - lr * cfg->weight_decay);
        t.init_npg[slot] = a.init_neg_pre_grad != 0 ? 1 : 0;
        t.vec[slot] = aligned16(a.param) && aligned16(a.grad) && aligned16(a.exp_avg) &&
                      aligned16(a.exp_avg_sq) && aligned16(a.exp_avg_diff) &&
                      aligned16(a.neg_pre_grad);
      },
      [&](const AdanTable& t, int blocks, int64_t) -> int {
        hipLaunchKernelGGL(k_adan, dim3(blocks), dim3(kOptThreads), 0, s, t, sc, grad_scale);
        HRF_LAUNCH_CHECK();
        return HRF_OK;
      });
}

int hrf_sparse_adam_update(float* param, const float* grad, float* exp_avg, float* exp_avg_sq,
                           const int64_t* visible, int64_t batch, int64_t rows, int64_t cols,
                           int64_t num_visible, float lr, float beta1, float beta2, float eps,
                           void* stream) {
  if (batch < 0 || rows < 0 || cols < 0 || num_visible < 0) {
    set_error("sparse adam: negative shape (%lld, %lld, %lld, %lld)",
              static_cast<long long>(batch), static_cast<long long>(rows),
              static_cast<long long>(cols), static_cast<long long>(num_visible));
    return HRF_ERR_INVALID;
  }
  const int64_t total = batch * num_visible * cols;
  if (total == 0) return HRF_OK;
  if (!param || !grad || !exp_avg || !exp_avg_sq || !visible) {
    set_error("sparse adam: null pointer");
    return HRF_ERR_INVALID;
  }
  if (total / kOptThreads >= 0x7FFFFFFFLL) {
    set_error("sparse adam: too many elements (%lld)", static_cast<long long>(total));
    return HRF_ERR_INVALID;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_sparse_adam, dim3(blocks_for(total, kOptThreads)), dim3(kOptThreads), 0,
                     s, param, grad, exp_avg, exp_avg_sq, visible, batch, rows, num_visible,
                     cols, lr, beta1, beta2, eps);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

}  // extern "C"
