// raster_render.hip — stage 3: tile-wise complex field compositing, forward
// (front to back) and backward (back to front), for gfx950.
//
// Work decomposition.  One 256-thread block (four wave64s, one pixel per
// lane) per (16x16 tile, depth plane).  The reference instead loops over the
// planes inside one block and re-scans the whole tile list per plane
// (forward_splat.cu:147-287, backward_splat.cu:131-306); here the planes run
// as independent blocks, so each plane terminates on its own and its blocks
// only touch that plane's Gaussians.  Per batch of 256 list entries a block
// ballot-compacts the entries whose plane weight passes the cutoff and stages
// their records (mean, conic, opacity, weight, complex amplitude) in LDS;
// every lane then reads each record with a uniform-address (broadcast) LDS
// load.  Blocks are mapped to (tile, plane) XCD-aware: the 8 XCDs receive
// blocks round-robin, so consecutive logical ids are given to one XCD and the
// P planes of a tile (and neighbouring tiles) share that XCD's L2.
//
// Backward gradients: per staged Gaussian each wave reduces its 6+2C partial
// sums with DPP (quad_perm, row mirrors, row_bcast15/31), accumulates the
// four wave totals with LDS float atomics, and one global atomic per
// (block, Gaussian, value) lands in a per-Gaussian accumulator.  The
// reference issues 8+2C global atomics per contributing (pixel, Gaussian).
#include "hrf_internal.h"

namespace hrf {
namespace {

__device__ __forceinline__ void map_block(int b, int nb, int P, int* tile, int* plane) {
  const int q = nb >> 3, r = nb & 7;
  const int x = b & 7, i = b >> 3;
  const int logical = (x < r) ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
  *tile = logical / P;
  *plane = logical - (*tile) * P;
}

// Tile range [r0, r0+n), clamped to the pair list so malformed caller input
// (the backward takes ranges from the caller) cannot index out of bounds.
__device__ __forceinline__ void tile_range(const RenderParams& p, int tile, int* r0, int* n) {
  const int64_t K = p.num_pairs;
  int64_t a = p.ranges[2 * tile], b = p.ranges[2 * tile + 1];
  a = a < 0 ? 0 : (a > K ? K : a);
  b = b < a ? a : (b > K ? K : b);
  *r0 = static_cast<int>(a);
  *n = static_cast<int>(b - a);
}

// exp(x) through the hardware base-2 exponential.
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, true));
}

// Wave64 sum; the total lands in lane 63.
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
  v += dpp_f<0xB1>(v);        // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);        // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);       // row_half_mirror
  v += dpp_f<0x140>(v);       // row_mirror
  v += dpp_f<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_f<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// Ballot compaction of one flag per thread across the block.  Returns the
// compacted position of this thread's entry and the block-wide count.
__device__ __forceinline__ int block_compact(bool flag, int* s_wt, int* count) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t bal = __ballot(flag);
  if (lane == 0) s_wt[wave] = __popcll(bal);
  __syncthreads();
  int off = 0, cnt = 0;
#pragma unroll
  for (int w = 0; w < kBlock / 64; ++w) {
    const int t = s_wt[w];
    off += (w < wave) ? t : 0;
    cnt += t;
  }
  *count = cnt;
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  return off + __popcll(bal & lt);
}

template <int C>
__global__ __launch_bounds__(kBlock) void k_render_fwd(RenderParams p) {
  constexpr int NQ = rec_quads(C);
  constexpr int RS = rec_stride(C);
  __shared__ float4 s_rec[kBlock * NQ];
  __shared__ int s_k[kBlock];
  __shared__ int s_wt[kBlock / 64];

  int tile, plane;
  map_block(blockIdx.x, gridDim.x, p.P, &tile, &plane);
  const int tx = tile % p.gx, ty = tile / p.gx;
  const int pxi = tx * kTile + (threadIdx.x & 15);
  const int pyi = ty * kTile + (threadIdx.x >> 4);
  const bool inside = pxi < p.W && pyi < p.H;
  int r0, n;
  tile_range(p, tile, &r0, &n);
  const float pxf = static_cast<float>(pxi), pyf = static_cast<float>(pyi);

  float T = 1.0f;
  float acc[2 * C];
#pragma unroll
  for (int i = 0; i < 2 * C; ++i) acc[i] = 0.0f;
  int last = 0;
  bool done = !inside;

  for (int base = 0; base < n; base += kBlock) {
    if (__syncthreads_and(done)) break;
    const int k = base + static_cast<int>(threadIdx.x);
    bool mem = false;
    int g = 0;
    if (k < n) {
      g = p.plist[r0 + k];
      mem = static_cast<uint64_t>(static_cast<uint32_t>(g)) < static_cast<uint64_t>(p.n) &&
            ((p.pmask[g] >> plane) & 1u);
    }
    int cnt;
    const int pos = block_compact(mem, s_wt, &cnt);
    if (mem) {
      const float4* src = reinterpret_cast<const float4*>(p.rec + static_cast<int64_t>(g) * RS);
#pragma unroll
      for (int q = 0; q < NQ; ++q) s_rec[pos * NQ + q] = src[q];
      s_rec[pos * NQ + 1].w = p.pprobs[static_cast<int64_t>(g) * p.P + plane];
      s_k[pos] = k;
    }
    __syncthreads();
    if (!done) {
      for (int j = 0; j < cnt; ++j) {
        const float4 a = s_rec[j * NQ];
        const float4 b = s_rec[j * NQ + 1];
        const float dx = a.x - pxf, dy = a.y - pyf;
        const float power =
            -0.5f * fmaf(dx, fmaf(a.z, dx, b.x * dy), dy * fmaf(a.w, dx, b.y * dy));
        if (power > 0.0f) continue;
        const float G = fast_exp(power);
        const float alpha = fminf(kMaxAlpha, b.z * G * b.w);
        const float Tn = T * (1.0f - alpha);
        const float sT = alpha * T;
        float amp[8];
        {
          const float4 c0 = s_rec[j * NQ + 2];
          const float4 c1 = s_rec[j * NQ + (NQ > 3 ? 3 : 2)];
          amp[0] = c0.x;
          amp[1] = c0.y;
          amp[2] = c0.z;
          amp[3] = c0.w;
          amp[4] = c1.x;
          amp[5] = c1.y;
          amp[6] = c1.z;
          amp[7] = c1.w;
        }
#pragma unroll
        for (int c = 0; c < C; ++c) {
          acc[2 * c] = fmaf(sT, amp[2 * c], acc[2 * c]);
          acc[2 * c + 1] = fmaf(sT, amp[2 * c + 1], acc[2 * c + 1]);
        }
        T = Tn;
        last = s_k[j] + 1;
        if (Tn < kTermT) {
          done = true;
          break;
        }
      }
    }
  }

  if (inside) {
    const int64_t HW = static_cast<int64_t>(p.W) * p.H;
    const int64_t pix = static_cast<int64_t>(pyi) * p.W + pxi;
#pragma unroll
    for (int c = 0; c < C; ++c)
      p.field[(static_cast<int64_t>(plane) * C + c) * HW + pix] = make_float2(acc[2 * c], acc[2 * c + 1]);
    p.final_T[plane * HW + pix] = T;
    p.n_contrib[plane * HW + pix] = last;
  }
}

template <int C>
__global__ __launch_bounds__(kBlock) void k_render_bwd(RenderParams p) {
  constexpr int NQ = rec_quads(C);
  constexpr int RS = rec_stride(C);
  constexpr int NV = 6 + 2 * C;
  __shared__ float4 s_rec[kBlock * NQ];
  __shared__ int s_k[kBlock];
  __shared__ int s_g[kBlock];
  __shared__ float s_acc[kBlock * NV];
  __shared__ int s_wt[kBlock / 64];
  __shared__ int s_maxlast;

  int tile, plane;
  map_block(blockIdx.x, gridDim.x, p.P, &tile, &plane);
  const int tx = tile % p.gx, ty = tile / p.gx;
  const int pxi = tx * kTile + (threadIdx.x & 15);
  const int pyi = ty * kTile + (threadIdx.x >> 4);
  const bool inside = pxi < p.W && pyi < p.H;
  int r0, n;
  tile_range(p, tile, &r0, &n);
  const float pxf = static_cast<float>(pxi), pyf = static_cast<float>(pyi);
  const int64_t HW = static_cast<int64_t>(p.W) * p.H;
  const int64_t pix = static_cast<int64_t>(pyi) * p.W + pxi;
  const int lane = threadIdx.x & 63;
  const int AS = acc_stride(C, p.P);

  float T = 0.0f;
  int last = 0;
  float gre[C], gim[C];
#pragma unroll
  for (int c = 0; c < C; ++c) gre[c] = gim[c] = 0.0f;
  if (inside) {
    T = p.final_T_in[plane * HW + pix];
    last = p.n_contrib_in[plane * HW + pix];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const float2 gv = p.grad_field[(static_cast<int64_t>(plane) * C + c) * HW + pix];
      gre[c] = gv.x;
      gim[c] = gv.y;
    }
  }
  if (threadIdx.x == 0) s_maxlast = 0;
  __syncthreads();
  if (inside && last > 0) atomicMax(&s_maxlast, last);
  __syncthreads();
  const int maxlast = s_maxlast < n ? s_maxlast : n;

  float accr[C], acci[C], lastr[C], lasti[C];
#pragma unroll
  for (int c = 0; c < C; ++c) accr[c] = acci[c] = lastr[c] = lasti[c] = 0.0f;
  float last_alpha = 0.0f;
  const float half_w = 0.5f * static_cast<float>(p.W);
  const float half_h = 0.5f * static_cast<float>(p.H);

  for (int end = maxlast; end > 0; end -= kBlock) {
    const int start = end > kBlock ? end - kBlock : 0;
    __syncthreads();
    const int k = start + static_cast<int>(threadIdx.x);
    bool mem = false;
    int g = 0;
    if (k < end) {
      g = p.plist[r0 + k];
      mem = static_cast<uint64_t>(static_cast<uint32_t>(g)) < static_cast<uint64_t>(p.n) &&
            ((p.pmask[g] >> plane) & 1u);
    }
    int cnt;
    const int pos = block_compact(mem, s_wt, &cnt);
    if (mem) {
      const float4* src = reinterpret_cast<const float4*>(p.rec + static_cast<int64_t>(g) * RS);
#pragma unroll
      for (int q = 0; q < NQ; ++q) s_rec[pos * NQ + q] = src[q];
      s_rec[pos * NQ + 1].w = p.pprobs[static_cast<int64_t>(g) * p.P + plane];
      s_k[pos] = k;
      s_g[pos] = g;
    }
    for (int e = threadIdx.x; e < cnt * NV; e += kBlock) s_acc[e] = 0.0f;
    __syncthreads();

    for (int j = cnt - 1; j >= 0; --j) {
      float v[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) v[i] = 0.0f;
      bool con = false;
      if (inside && s_k[j] < last) {
        const float4 a = s_rec[j * NQ];
        const float4 b = s_rec[j * NQ + 1];
        const float dx = a.x - pxf, dy = a.y - pyf;
        const float cxx = a.z, cxy = a.w, czz = b.y;
        const float power = -0.5f * (cxx * dx * dx + czz * dy * dy) - cxy * dx * dy;
        if (power <= 0.0f) {
          const float G = fast_exp(power);
          const float alpha = fminf(kMaxAlpha, b.z * G * b.w);
          if (alpha >= kMinAlphaBwd) {
            T = T / (1.0f - alpha);
            const float dcol = alpha * T;
            float amp[8];
            {
              const float4 c0 = s_rec[j * NQ + 2];
              amp[0] = c0.x;
              amp[1] = c0.y;
              amp[2] = c0.z;
              amp[3] = c0.w;
              const float4 c1 = s_rec[j * NQ + (NQ > 3 ? 3 : 2)];
              amp[4] = c1.x;
              amp[5] = c1.y;
              amp[6] = c1.z;
              amp[7] = c1.w;
            }
            float dLda = 0.0f;
#pragma unroll
            for (int c = 0; c < C; ++c) {
              const float cr = amp[2 * c], ci = amp[2 * c + 1];
              accr[c] = last_alpha * lastr[c] + (1.0f - last_alpha) * accr[c];
              acci[c] = last_alpha * lasti[c] + (1.0f - last_alpha) * acci[c];
              lastr[c] = cr;
              lasti[c] = ci;
              dLda += (cr - accr[c]) * gre[c];
              dLda += (ci - acci[c]) * gim[c];
              v[6 + c] = dcol * gre[c];
              v[6 + C + c] = dcol * gim[c];
            }
            dLda *= T;
            last_alpha = alpha;
            const float Q = G * dLda;
            v[0] = Q * fmaf(dx, cxx, dy * cxy);
            v[1] = Q * fmaf(dy, czz, dx * cxy);
            v[2] = Q * dx * dx;
            v[3] = Q * dx * dy;
            v[4] = Q * dy * dy;
            v[5] = Q;
            con = true;
          }
        }
      }
      if (__ballot(con) != 0ull) {
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] = wave_sum_to_lane63(v[i]);
        if (lane == 63) {
#pragma unroll
          for (int i = 0; i < NV; ++i) atomicAdd(&s_acc[j * NV + i], v[i]);
        }
      }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < cnt * NV; e += kBlock) {
      const float val = s_acc[e];
      if (val == 0.0f) continue;
      const int j = e / NV, i = e - j * NV;
      const int gg = s_g[j];
      const float4 b = s_rec[j * NQ + 1];
      const float ow = b.z * b.w;
      int slot;
      float scale;
      if (i == 0) {
        slot = 0;
        scale = -half_w * ow;
      } else if (i == 1) {
        slot = 1;
        scale = -half_h * ow;
      } else if (i < 5) {
        slot = i;
        scale = -0.5f * ow;
      } else if (i == 5) {
        slot = 5 + 2 * C + plane;
        scale = 1.0f;
      } else {
        slot = i - 1;  // A_c at 5+c (i = 6+c), B_c at 5+C+c (i = 6+C+c)
        scale = 1.0f;
      }
      unsafeAtomicAdd(p.acc + static_cast<int64_t>(gg) * AS + slot, val * scale);
    }
  }
}

__global__ void k_render_empty(float2* field, float* final_T, int32_t* n_contrib,
                               int64_t npix, int PC, int P) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < npix * PC) field[i] = make_float2(0.0f, 0.0f);
  if (i < npix * P) {
    final_T[i] = 1.0f;
    n_contrib[i] = 0;
  }
}

}  // namespace

int launch_render_forward(const RenderParams& p, hipStream_t s) {
  const int nblocks = p.gx * p.gy * p.P;
  if (nblocks <= 0) return HRF_OK;
  switch (p.C) {
    case 1:
      hipLaunchKernelGGL(k_render_fwd<1>, dim3(nblocks), dim3(kBlock), 0, s, p);
      break;
    case 2:
      hipLaunchKernelGGL(k_render_fwd<2>, dim3(nblocks), dim3(kBlock), 0, s, p);
      break;
    case 3:
      hipLaunchKernelGGL(k_render_fwd<3>, dim3(nblocks), dim3(kBlock), 0, s, p);
      break;
    default:
      set_error("render: channels must be 1..3 (got %d)", p.C);
      return HRF_ERR_INVALID;
  }
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_render_backward(const RenderParams& p, hipStream_t s) {
  const int nblocks = p.gx * p.gy * p.P;
  if (nblocks <= 0) return HRF_OK;
  switch (p.C) {
    case 1:
      hipLaunchKernelGGL(k_render_bwd<1>, dim3(nblocks), dim3(kBlock), 0, s, p);
      break;
    case 2:
      hipLaunchKernelGGL(k_render_bwd<2>, dim3(nblocks), dim3(kBlock), 0, s, p);
      break;
    case 3:
      hipLaunchKernelGGL(k_render_bwd<3>, dim3(nblocks), dim3(kBlock), 0, s, p);
      break;
    default:
      set_error("render backward: channels must be 1..3 (got %d)", p.C);
      return HRF_ERR_INVALID;
  }
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_render_empty(const RenderParams& p, hipStream_t s) {
  const int64_t npix = static_cast<int64_t>(p.W) * p.H;
  const int64_t total = npix * (p.P * p.C > p.P ? p.P * p.C : p.P);
  if (total <= 0) return HRF_OK;
  hipLaunchKernelGGL(k_render_empty, dim3(blocks_for(total, 256)), dim3(256), 0, s, p.field,
                     p.final_T, p.n_contrib, npix, p.P * p.C, p.P);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

}  // namespace hrf
