// preprocess.hip — the caller-side glue of Scene.render ahead of the
// rasterizer, fused: world -> camera transform, near/far + z >= 0 filter,
// ascending depth order, the gathers and the parameter activations, and the
// backward of all of it (scatter back to the N parameter rows).
//
// Reference: Scene.render (model.py:1365-1402), compute_depth_values
// (model.py:1105-1112), get_idxs_to_filter_and_sort (model.py:1121-1125),
// Gaussians.apply_activations (model.py:594-608), STEFunction
// (model.py:41-56), and the transform in Scene.splat (model.py:1161-1162).
// The reference runs ~15 torch ops and a global torch.sort; here the
// selection is one kernel over the parameters in index order (transform,
// filter and every activation, packed into one record per kept row), the
// flag scan shared with the binning, one compaction, a stable 32-bit radix
// sort of the selected depth keys, and one gather of the records in depth
// order.  The backward packs the output gradients in depth order, then
// writes every parameter-gradient row in index order, so both passes over
// the parameter arrays are coalesced.
#include <cmath>

#include "hrf_internal.h"

namespace hrf {
namespace {

constexpr int kPreThreads = 256;

struct View {
  float r[9];  // R row-major: cam_j = sum_i m_i R[i][j] + T[j]
  float t[3];
};

__device__ __forceinline__ View load_view(const float* __restrict__ R,
                                          const float* __restrict__ T) {
  View v;
#pragma unroll
  for (int i = 0; i < 9; ++i) v.r[i] = R[i];
#pragma unroll
  for (int i = 0; i < 3; ++i) v.t[i] = T[i];
  return v;
}

// X_cam = X_world @ R + T, left to right without contraction
// (model.py:1110: means_3D @ R + T; pytorch3d's world-to-view transform of
// Scene.splat computes the same product).
__device__ __forceinline__ void to_camera(const View& v, float m0, float m1, float m2,
                                          float* c) {
#pragma unroll
  for (int j = 0; j < 3; ++j) c[j] = m0 * v.r[j] + m1 * v.r[3 + j] + m2 * v.r[6 + j] + v.t[j];
}

// Packed per-Gaussian records.  The selection pass reads every parameter
// row in index order (coalesced) and writes, for each kept Gaussian, one
// record with everything the depth-ordered gather needs, so the gather reads
// one contiguous record per row instead of seven scattered ones:
//   [cam 3 | quat 4 | scale 3 | opacity | plane index (int bits) | colour C | phase C]
// The backward packs the M output-gradient rows the same way, in depth order:
//   [cam 3 (+ z) | quat 4 | scale 3 | opacity | colour C | phase C | plane P]
// and a second pass in parameter order reads its row's record.
__host__ __device__ constexpr int round4(int x) { return (x + 3) & ~3; }
__host__ __device__ constexpr int fwd_stride(int C) { return round4(12 + 2 * C); }
__host__ __device__ constexpr int bwd_stride(int C, int P) { return round4(11 + 2 * C + P); }

constexpr uint32_t kNotSelected = 0xFFFFFFFFu;

// Registers of one record when its stride is a compile-time constant (kS > 0):
// filled or drained with 16-byte accesses; with kS == 0 every element goes
// straight to or from memory.
template <int kS>
struct Rec {
  float v[kS > 0 ? kS : 1] = {};
  float* mem;
  __device__ __forceinline__ explicit Rec(float* p) : mem(p) {}
  __device__ __forceinline__ void put(int k, float x) {
    if constexpr (kS > 0) v[k] = x; else mem[k] = x;
  }
  __device__ __forceinline__ float get(int k) const {
    if constexpr (kS > 0) return v[k]; else return mem[k];
  }
  __device__ __forceinline__ void store() {
    if constexpr (kS > 0) {
#pragma unroll
      for (int k = 0; k < kS; k += 4)
        *reinterpret_cast<float4*>(mem + k) = make_float4(v[k], v[k + 1], v[k + 2], v[k + 3]);
    }
  }
  __device__ __forceinline__ void load() {
    if constexpr (kS > 0) {
#pragma unroll
      for (int k = 0; k < kS; k += 4) {
        const float4 q = *reinterpret_cast<const float4*>(mem + k);
        v[k] = q.x;
        v[k + 1] = q.y;
        v[k + 2] = q.z;
        v[k + 3] = q.w;
      }
    }
  }
};

// torch.remainder(x, 2*pi) with the divisor as float32: fmod (exact), then
// the sign of the divisor (model.py:602).
__device__ __forceinline__ float remainder_2pi(float x) {
  const float b = 6.28318530717958647692f;
  float r = fmodf(x, b);
  if (r != 0.0f && (r < 0.0f) != (b < 0.0f)) r += b;
  return r;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// Selection flag and depth sort key of every Gaussian: kept when
// near < z < far (model.py:1382-1385) and z >= 0 (model.py:1123); the key
// orders non-negative floats (-0 counts as 0).  A kept Gaussian's record
// carries its activations (model.py:594-608): F.normalize(q) with eps 1e-12,
// exp(log-scales), sigmoid(opacity), colours, phase mod 2*pi and the
// argmax plane (first maximal entry, NaN counting as the maximum).
template <int kC>
__global__ __launch_bounds__(kPreThreads) void k_pre_select(
    hrf_scene_params sp, const float* __restrict__ R, const float* __restrict__ T,
    float near_plane, float far_plane, uint32_t* __restrict__ flag, uint32_t* __restrict__ key,
    float* __restrict__ rec) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= sp.n) return;
  const View v = load_view(R, T);
  float c[3];
  to_camera(v, sp.means[3 * g], sp.means[3 * g + 1], sp.means[3 * g + 2], c);
  const float z = c[2];
  const bool keep = z > near_plane && z < far_plane && z >= 0.0f;
  flag[g] = keep ? 1u : 0u;
  key[g] = __float_as_uint(z) & 0x7FFFFFFFu;
  if (!keep) return;
  const int C = kC > 0 ? kC : sp.channels, P = sp.planes;
  Rec<(kC > 0 ? fwd_stride(kC) : 0)> r(rec + g * fwd_stride(C));
  r.put(0, c[0]);
  r.put(1, c[1]);
  r.put(2, c[2]);
  const float q0 = sp.pre_quats[4 * g], q1 = sp.pre_quats[4 * g + 1];
  const float q2 = sp.pre_quats[4 * g + 2], q3 = sp.pre_quats[4 * g + 3];
  const float nrm = fmaxf(sqrtf(q0 * q0 + q1 * q1 + q2 * q2 + q3 * q3), 1e-12f);
  r.put(3, q0 / nrm);
  r.put(4, q1 / nrm);
  r.put(5, q2 / nrm);
  r.put(6, q3 / nrm);
#pragma unroll
  for (int j = 0; j < 3; ++j) r.put(7 + j, expf(sp.pre_scales[3 * g + j]));
  r.put(10, sigmoidf_(sp.pre_opacities[g]));
  int best = 0;
  float bv = sp.pre_plane[g * P];
  for (int p = 1; p < P; ++p) {
    const float x = sp.pre_plane[g * P + p];
    if (!(bv != bv) && (x > bv || x != x)) {
      bv = x;
      best = p;
    }
  }
  r.put(11, __int_as_float(best));
#pragma unroll
  for (int j = 0; j < C; ++j) {
    r.put(12 + j, sp.colours[g * C + j]);
    r.put(12 + C + j, remainder_2pi(sp.pre_phase[g * C + j]));
  }
  r.store();
}

__global__ __launch_bounds__(kPreThreads) void k_pre_compact(
    const uint32_t* __restrict__ flag, const uint32_t* __restrict__ pos,
    const uint32_t* __restrict__ key, int64_t n, uint32_t* __restrict__ ckey,
    uint32_t* __restrict__ cidx) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n || !flag[g]) return;
  const uint32_t p = pos[g];
  ckey[p] = key[g];
  cidx[p] = static_cast<uint32_t>(g);
}

// The m selected Gaussians in depth order: one record read per row, the
// rasterizer inputs written row-contiguous.
template <int kC>
__global__ __launch_bounds__(kPreThreads) void k_pre_gather(
    const float* __restrict__ rec, int channels, int P, const uint32_t* __restrict__ sidx,
    int64_t m, float* __restrict__ cam, float* __restrict__ zv, float* __restrict__ quats,
    float* __restrict__ scales, float* __restrict__ colours, float* __restrict__ phase,
    float* __restrict__ opac, float* __restrict__ pprobs, int64_t* __restrict__ idxs) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= m) return;
  const int64_t g = sidx[i];
  const int C = kC > 0 ? kC : channels;
  Rec<(kC > 0 ? fwd_stride(kC) : 0)> r(const_cast<float*>(rec) + g * fwd_stride(C));
  r.load();
#pragma unroll
  for (int j = 0; j < 3; ++j) cam[3 * i + j] = r.get(j);
  zv[i] = r.get(2);
#pragma unroll
  for (int j = 0; j < 4; ++j) quats[4 * i + j] = r.get(3 + j);
#pragma unroll
  for (int j = 0; j < 3; ++j) scales[3 * i + j] = r.get(7 + j);
  opac[i] = r.get(10);
  const int best = __float_as_int(r.get(11));
#pragma unroll
  for (int j = 0; j < C; ++j) {
    colours[i * C + j] = r.get(12 + j);
    phase[i * C + j] = r.get(12 + C + j);
  }
  for (int p = 0; p < P; ++p) pprobs[i * P + p] = p == best ? 1.0f : 0.0f;
  idxs[i] = g;
}

// Backward, pass 1 (depth order): pack the output-gradient rows of each
// selected Gaussian and record its position under its parameter row.
template <int kC, int kP>
__global__ __launch_bounds__(kPreThreads) void k_pre_bpack(
    const int64_t* __restrict__ idxs, int64_t m, int64_t n, int channels, int planes,
    hrf_selected_grads gin, float* __restrict__ grec, uint32_t* __restrict__ inv) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= m) return;
  const int64_t g = idxs[i];
  if (g < 0 || g >= n) return;
  const int C = kC > 0 ? kC : channels, P = kP > 0 ? kP : planes;
  Rec<(kC > 0 && kP > 0 ? bwd_stride(kC, kP) : 0)> r(grec + i * bwd_stride(C, P));
  r.put(0, gin.cam[3 * i]);
  r.put(1, gin.cam[3 * i + 1]);
  r.put(2, gin.cam[3 * i + 2] + (gin.z ? gin.z[i] : 0.0f));
#pragma unroll
  for (int j = 0; j < 4; ++j) r.put(3 + j, gin.quats[4 * i + j]);
#pragma unroll
  for (int j = 0; j < 3; ++j) r.put(7 + j, gin.scales[3 * i + j]);
  r.put(10, gin.opacities[i]);
#pragma unroll
  for (int j = 0; j < C; ++j) {
    r.put(11 + j, gin.colours[i * C + j]);
    r.put(11 + C + j, gin.phase[i * C + j]);
  }
#pragma unroll
  for (int p = 0; p < P; ++p) r.put(11 + 2 * C + p, gin.plane_probs[i * P + p]);
  r.store();
  inv[g] = static_cast<uint32_t>(i);
}

// Backward, pass 2 (parameter order): every parameter-gradient row, zero for
// rows that were not selected.  cam = m @ R + T and z = cam.z give
// d m_k = sum_j g_cam_j R[k][j] + g_z R[k][2]; F.normalize gives
// (g - y (y . g)) / ||q|| above eps and g / eps below; exp and sigmoid use
// their outputs; STEFunction.backward is grad * softmax(x / 0.001)
// (model.py:50-56).
template <int kC, int kP>
__global__ __launch_bounds__(kPreThreads) void k_pre_bscatter(
    hrf_scene_params sp, const float* __restrict__ R, const uint32_t* __restrict__ inv,
    const float* __restrict__ grec, hrf_param_grads d) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= sp.n) return;
  const int C = kC > 0 ? kC : sp.channels, P = kP > 0 ? kP : sp.planes;
  const uint32_t i = inv[g];
  if (i == kNotSelected) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      d.means[3 * g + j] = 0.0f;
      d.pre_scales[3 * g + j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) d.pre_quats[4 * g + j] = 0.0f;
#pragma unroll
    for (int j = 0; j < C; ++j) {
      d.colours[g * C + j] = 0.0f;
      d.pre_phase[g * C + j] = 0.0f;
    }
    d.pre_opacities[g] = 0.0f;
#pragma unroll
    for (int p = 0; p < P; ++p) d.pre_plane[g * P + p] = 0.0f;
    return;
  }
  Rec<(kC > 0 && kP > 0 ? bwd_stride(kC, kP) : 0)> r(
      const_cast<float*>(grec) + static_cast<int64_t>(i) * bwd_stride(C, P));
  r.load();
  const float gc0 = r.get(0), gc1 = r.get(1), gc2 = r.get(2);
#pragma unroll
  for (int k = 0; k < 3; ++k)
    d.means[3 * g + k] = gc0 * R[3 * k] + gc1 * R[3 * k + 1] + gc2 * R[3 * k + 2];
  const float q0 = sp.pre_quats[4 * g], q1 = sp.pre_quats[4 * g + 1];
  const float q2 = sp.pre_quats[4 * g + 2], q3 = sp.pre_quats[4 * g + 3];
  const float raw = sqrtf(q0 * q0 + q1 * q1 + q2 * q2 + q3 * q3);
  const float gq[4] = {r.get(3), r.get(4), r.get(5), r.get(6)};
  if (raw > 1e-12f) {
    const float y[4] = {q0 / raw, q1 / raw, q2 / raw, q3 / raw};
    const float dot = y[0] * gq[0] + y[1] * gq[1] + y[2] * gq[2] + y[3] * gq[3];
#pragma unroll
    for (int j = 0; j < 4; ++j) d.pre_quats[4 * g + j] = (gq[j] - y[j] * dot) / raw;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) d.pre_quats[4 * g + j] = gq[j] / 1e-12f;
  }
#pragma unroll
  for (int j = 0; j < 3; ++j)
    d.pre_scales[3 * g + j] = r.get(7 + j) * expf(sp.pre_scales[3 * g + j]);
  const float s = sigmoidf_(sp.pre_opacities[g]);
  d.pre_opacities[g] = r.get(10) * (s * (1.0f - s));
#pragma unroll
  for (int j = 0; j < C; ++j) {
    d.colours[g * C + j] = r.get(11 + j);
    d.pre_phase[g * C + j] = r.get(11 + C + j);
  }
  float mx = -INFINITY;
#pragma unroll
  for (int p = 0; p < P; ++p) mx = fmaxf(mx, sp.pre_plane[g * P + p] / 0.001f);
  float den = 0.0f;
#pragma unroll
  for (int p = 0; p < P; ++p) den += expf(sp.pre_plane[g * P + p] / 0.001f - mx);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const float sm = expf(sp.pre_plane[g * P + p] / 0.001f - mx) / den;
    d.pre_plane[g * P + p] = r.get(11 + 2 * C + p) * sm;
  }
}

struct PreWs {
  uint32_t* flag;
  uint32_t* pos;
  uint32_t* key;
  uint32_t* ckey;
  uint32_t* cidx;
  uint32_t* ckey_b;
  uint32_t* cidx_b;
  uint64_t* off;
  uint64_t* bsum_p;
  uint32_t* bsum_v;
  uint32_t* zero;
  uint32_t* radix;
  float* rec;  // n records of fwd_stride(C) floats, written for kept rows
};

PreWs carve_pre(Carver& cv, int64_t n, int C) {
  PreWs w;
  const int64_t m = n > 0 ? n : 1;
  w.flag = cv.take<uint32_t>(m);
  w.pos = cv.take<uint32_t>(m);
  w.key = cv.take<uint32_t>(m);
  w.ckey = cv.take<uint32_t>(m);
  w.cidx = cv.take<uint32_t>(m);
  w.ckey_b = cv.take<uint32_t>(m);
  w.cidx_b = cv.take<uint32_t>(m);
  w.off = cv.take<uint64_t>(m + 1);
  w.bsum_p = cv.take<uint64_t>(scan_scratch_elems(m));
  w.bsum_v = cv.take<uint32_t>(scan_scratch_elems(m));
  w.zero = cv.take<uint32_t>(4);
  w.radix = cv.take<uint32_t>(radix_scratch_elems(m));
  w.rec = cv.take<float>(m * fwd_stride(C));
  return w;
}

// The backward's layout of the same workspace (nothing carries over from
// the forward): the position of each parameter row in depth order
// (kNotSelected if it was not selected) and the packed gradient records.
struct PreBwdWs {
  uint32_t* inv;
  float* grec;
};

PreBwdWs carve_pre_bwd(Carver& cv, int64_t n, int C, int P) {
  PreBwdWs w;
  const int64_t m = n > 0 ? n : 1;
  w.inv = cv.take<uint32_t>(m);
  w.grec = cv.take<float>(m * bwd_stride(C, P));
  return w;
}

size_t pre_ws_bytes(int64_t n, int C, int P) {
  Carver f(nullptr), b(nullptr);
  carve_pre(f, n, C);
  carve_pre_bwd(b, n, C, P);
  return f.bytes() > b.bytes() ? f.bytes() : b.bytes();
}

int check_params(const hrf_scene_params* sp) {
  if (!sp || sp->n < 0 || sp->channels < 1 || sp->planes < 1 || sp->planes > kMaxPlanes) {
    set_error("preprocess: invalid parameters (need n >= 0, channels >= 1, planes 1..%d)",
              kMaxPlanes);
    return HRF_ERR_INVALID;
  }
  if (sp->n > 0 && (!sp->means || !sp->pre_quats || !sp->pre_scales || !sp->colours ||
                    !sp->pre_phase || !sp->pre_opacities || !sp->pre_plane)) {
    set_error("preprocess: null parameter pointer");
    return HRF_ERR_INVALID;
  }
  if (sp->n > 0x7FFFFFFFLL) {
    set_error("preprocess: %lld Gaussians exceed the 32-bit index range",
              static_cast<long long>(sp->n));
    return HRF_ERR_INVALID;
  }
  return HRF_OK;
}

}  // namespace
}  // namespace hrf

using namespace hrf;

extern "C" {

size_t hrf_preprocess_workspace_size(int64_t n, int32_t channels, int32_t planes) {
  if (n < 0 || channels < 1 || planes < 1) return 0;
  return pre_ws_bytes(n, channels, planes);
}

int hrf_preprocess_select(const hrf_scene_params* sp, const float* R, const float* T,
                          float near_plane, float far_plane, void* ws, size_t ws_bytes,
                          void* stream, int64_t* num_selected) {
  HRF_TRY(check_params(sp));
  if (!num_selected || !R || !T) {
    set_error("preprocess: null R/T or count output");
    return HRF_ERR_INVALID;
  }
  *num_selected = 0;
  const int64_t n = sp->n;
  if (n == 0) return HRF_OK;
  const size_t need = pre_ws_bytes(n, sp->channels, sp->planes);
  if (!ws || ws_bytes < need) {
    set_error("preprocess workspace too small: %zu bytes given, %zu needed", ws_bytes, need);
    return HRF_ERR_WORKSPACE;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  Carver cv(ws);
  PreWs w = carve_pre(cv, n, sp->channels);
  ReadbackSlot slot;
  HRF_TRY(readback_acquire(&slot.r));
  const uint64_t tag = readback_arm(slot.r);
  HRF_STAGE("pre_select", s);
  HRF_TRY(launch_fill_u32(w.zero, 0u, 1, s));
  const dim3 grid(blocks_for(n, kPreThreads));
  if (sp->channels == 3)
    hipLaunchKernelGGL(k_pre_select<3>, grid, dim3(kPreThreads), 0, s, *sp, R, T, near_plane,
                       far_plane, w.flag, w.key, w.rec);
  else
    hipLaunchKernelGGL(k_pre_select<0>, grid, dim3(kPreThreads), 0, s, *sp, R, T, near_plane,
                       far_plane, w.flag, w.key, w.rec);
  HRF_LAUNCH_CHECK();
  // Exclusive positions of the kept Gaussians (the binning's offsets scan,
  // with the flags as both of its inputs); totals[1] = kept count, written
  // into the pinned read-back words, read while the compaction runs.
  slot.pending = true;
  HRF_TRY(launch_offsets(nullptr, w.flag, w.flag, n, w.off, w.pos, w.bsum_p, w.bsum_v, w.zero,
                         slot.r->dev, s, tag));
  hipLaunchKernelGGL(k_pre_compact, grid, dim3(kPreThreads), 0, s, w.flag, w.pos, w.key, n,
                     w.ckey, w.cidx);
  HRF_LAUNCH_CHECK();
  HRF_TRY(readback_wait(slot.r, tag, s));
  slot.pending = false;
  const uint64_t kept = slot.r->host[1];
  if (kept > static_cast<uint64_t>(n)) {
    set_error("internal: selection count read-back incomplete (%llu)",
              static_cast<unsigned long long>(kept));
    return HRF_ERR_INVALID;
  }
  const int64_t m = static_cast<int64_t>(kept);
  if (m > 1) {
    // Stable ascending depth order (ties keep index order); 4 passes, so
    // the result ends in (ckey, cidx).
    bool in_b = false;
    HRF_TRY(radix_sort_pairs(w.ckey, w.cidx, w.ckey_b, w.cidx_b, m, 32, w.radix, &in_b, s));
    if (in_b) {
      set_error("internal: preprocess sort expected an even pass count");
      return HRF_ERR_INVALID;
    }
  }
  *num_selected = m;
  return HRF_OK;
}

int hrf_preprocess_forward(const hrf_scene_params* sp, const float* R, const float* T,
                           const void* ws, size_t ws_bytes, int64_t num_selected,
                           float* cam_means, float* z_vals, float* quats, float* scales,
                           float* colours, float* phase, float* opacities, float* plane_probs,
                           int64_t* idxs, void* stream) {
  HRF_TRY(check_params(sp));
  const int64_t m = num_selected;
  if (m < 0 || m > sp->n) {
    set_error("preprocess: invalid selected count %lld", static_cast<long long>(m));
    return HRF_ERR_INVALID;
  }
  if (m == 0) return HRF_OK;
  if (!R || !T || !cam_means || !z_vals || !quats || !scales || !colours || !phase ||
      !opacities || !plane_probs || !idxs) {
    set_error("preprocess: null output pointer");
    return HRF_ERR_INVALID;
  }
  const size_t need = pre_ws_bytes(sp->n, sp->channels, sp->planes);
  if (!ws || ws_bytes < need) {
    set_error("preprocess workspace too small: %zu bytes given, %zu needed", ws_bytes, need);
    return HRF_ERR_WORKSPACE;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  Carver cv(const_cast<void*>(ws));
  PreWs w = carve_pre(cv, sp->n, sp->channels);
  HRF_STAGE("pre_gather", s);
  const dim3 grid(blocks_for(m, kPreThreads));
  if (sp->channels == 3)
    hipLaunchKernelGGL(k_pre_gather<3>, grid, dim3(kPreThreads), 0, s, w.rec, sp->channels,
                       sp->planes, w.cidx, m, cam_means, z_vals, quats, scales, colours, phase,
                       opacities, plane_probs, idxs);
  else
    hipLaunchKernelGGL(k_pre_gather<0>, grid, dim3(kPreThreads), 0, s, w.rec, sp->channels,
                       sp->planes, w.cidx, m, cam_means, z_vals, quats, scales, colours, phase,
                       opacities, plane_probs, idxs);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int hrf_preprocess_backward(const hrf_scene_params* sp, const float* R, const int64_t* idxs,
                            int64_t num_selected, const hrf_selected_grads* grads,
                            const hrf_param_grads* out, void* ws, size_t ws_bytes,
                            void* stream) {
  HRF_TRY(check_params(sp));
  if (!grads || !out || !out->means || !out->pre_quats || !out->pre_scales || !out->colours ||
      !out->pre_phase || !out->pre_opacities || !out->pre_plane) {
    set_error("preprocess backward: null gradient pointer");
    return HRF_ERR_INVALID;
  }
  const int64_t n = sp->n, m = num_selected;
  if (m < 0 || m > n) {
    set_error("preprocess backward: invalid selected count %lld", static_cast<long long>(m));
    return HRF_ERR_INVALID;
  }
  if (n == 0) return HRF_OK;
  if (m > 0 && (!R || !idxs || !grads->cam || !grads->quats || !grads->scales ||
                !grads->colours || !grads->phase || !grads->opacities ||
                !grads->plane_probs)) {
    set_error("preprocess backward: null input pointer");
    return HRF_ERR_INVALID;
  }
  const size_t need = pre_ws_bytes(n, sp->channels, sp->planes);
  if (!ws || ws_bytes < need) {
    set_error("preprocess workspace too small: %zu bytes given, %zu needed", ws_bytes, need);
    return HRF_ERR_WORKSPACE;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  Carver cv(ws);
  PreBwdWs w = carve_pre_bwd(cv, n, sp->channels, sp->planes);
  const bool fast = sp->channels == 3 && sp->planes == 3;
  HRF_STAGE("pre_backward", s);
  HRF_TRY(launch_fill_u32(w.inv, kNotSelected, n, s));
  if (m > 0) {
    const dim3 grid(blocks_for(m, kPreThreads));
    if (fast)
      hipLaunchKernelGGL((k_pre_bpack<3, 3>), grid, dim3(kPreThreads), 0, s, idxs, m, n,
                         sp->channels, sp->planes, *grads, w.grec, w.inv);
    else
      hipLaunchKernelGGL((k_pre_bpack<0, 0>), grid, dim3(kPreThreads), 0, s, idxs, m, n,
                         sp->channels, sp->planes, *grads, w.grec, w.inv);
    HRF_LAUNCH_CHECK();
  }
  const dim3 grid(blocks_for(n, kPreThreads));
  if (fast)
    hipLaunchKernelGGL((k_pre_bscatter<3, 3>), grid, dim3(kPreThreads), 0, s, *sp, R, w.inv,
                       w.grec, *out);
  else
    hipLaunchKernelGGL((k_pre_bscatter<0, 0>), grid, dim3(kPreThreads), 0, s, *sp, R, w.inv,
                       w.grec, *out);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

}  // extern "C"
