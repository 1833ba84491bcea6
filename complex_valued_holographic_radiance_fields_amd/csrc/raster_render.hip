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
// blocks round-robin, so runs of consecutive tiles (all their planes) are
// given to one XCD and share its L2, while the runs interleave over the XCDs
// so that every XCD gets an even share of the dense image regions.
//
// Backward gradients: waves own 8x8 quadrants; each batch stages records
// with a per-quadrant cull mask (exact: alpha >= 1/255 box and n_contrib
// bound), each wave walks its own compacted list back to front and reduces
// the 6+2C per-lane partial sums of G members at once with a 64-value
// transpose-reduce (v_permlane32/16_swap + DPP), lands the totals in LDS
// with one ds_add per lane, and flushes one global atomic per (block,
// Gaussian, value) into a per-Gaussian accumulator.  The reference issues
// 8+2C global atomics per contributing (pixel, Gaussian).
#include <type_traits>

#include "hrf_internal.h"
#include "render_cull.h"
#include "render_member.h"
#include "wave_reduce.h"

namespace hrf {
namespace {

// Hardware block b runs on XCD b % 8.  Logical ids (tile-major, planes
// innermost) are dealt to the XCDs in runs of kRunTiles tiles: each XCD
// receives whole runs (neighbouring tiles share Gaussians in its L2), and
// the runs of all 8 XCDs advance together through the image, so the dense
// rows of a scene are spread over every XCD instead of loading a few.
constexpr int kRunTiles = 4;

__device__ __forceinline__ void map_block(int b, int nb, int P, int* tile, int* plane) {
  const int c = kRunTiles * P;  // logical ids per run
  const int full = nb - nb % (8 * c);
  int logical = b;
  if (b < full) {
    const int x = b & 7, i = b >> 3;
    const int run = i / c, off = i - run * c;
    logical = (run * 8 + x) * c + off;
  }
  *tile = logical / P;
  *plane = logical - (*tile) * P;
}

// Number of set bits of a wave mask below the calling lane (v_mbcnt).
__device__ __forceinline__ int bits_below_lane(uint64_t m) {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(
      static_cast<uint32_t>(m >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
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

// -log2(e)/2: the render kernels stage the conic pre-scaled by it, so the
// Gaussian's exponent comes out in base 2 with the -1/2 folded in.
constexpr float kBwdConicScale = -0.72134752044448170368f;
constexpr float kLog2E = 1.44269504088896340736f;

// Members per chunk of the backward's two-phase member walk.
constexpr int kBwdChunk = 4;

// a / b for b in [0.01, 1] and a normal: the hardware reciprocal, then one
// residual correction (the residual a - q b is exact in a fused
// multiply-add), which rounds like the reference's IEEE division
// (backward_splat.cu:222) except in rare near-tie cases.  The backward
// recovers T by up to 1e5 such divisions in a row, so the reciprocal's own
// error (up to 1 ulp, not zero-mean) would drift T by more than 1e-4.
__device__ __forceinline__ float div_rn(float a, float b) {
  const float r = __builtin_amdgcn_rcpf(b);
  const float q = a * r;
  return fmaf(fmaf(-q, b, a), r, q);
}

// The forward's per-wave batch word: member count, two flags, and the count
// of members written to the plane member lists (bits 16-23).
constexpr int kWtCount = 0xFF;
constexpr int kWtUnsafe = 0x100;
constexpr int kWtDone = 0x200;
constexpr int kWtClamp = 0x400;

// A batch whose staged members all have o w <= kNoClampOw runs the fast
// loops without the reference's alpha = min(0.99, .) clamp: there the fast
// exponent is log2(o w) plus a quadratic form that is negative and rounds
// by far less than log2(0.99 / 0.98) (the 2-D covariance carries the +0.3
// dilation, so the conic is bounded), so exp2 of it stays below 0.99 and
// the clamp would return its argument unchanged.
constexpr float kNoClampOw = 0.98f;
constexpr int kWtSubShift = 16;

// List entries per window of the tagged forward walk (tag bytes scanned per
// compaction; positions within a window fit 16 bits).
constexpr int kTagWin = 2048;

// Plane member list entries: (gaussian, list position | quadrant mask << 28).
// The mask has bit w set when the member's alpha >= 1/255 region meets the
// 8x8 quadrant w of the tile (the backward's box test, made once in the
// forward); members meeting no quadrant are not listed.  List positions are
// below the Gaussian count, which the library keeps under 2^28 for lists.
constexpr int kSubPosBits = 28;
constexpr uint32_t kSubPosMask = (1u << kSubPosBits) - 1u;

// A conic the fast member loops may evaluate in their own form: positive
// definite with |correlation| below 0.99 (b b2 < 0.98 a c).  The exponent
// dx (A dx + B dy) + C dy^2 is a sum of terms at most (1 + r) / (1 - r) = 199
// times its value, so any evaluation order rounds it alike to within a few
// 1e-5 relative even in a Gaussian's far tail, and it cannot round to a
// positive value (the reference's "power > 0: skip" test never fires).  A
// batch that stages any other conic runs the exact loop, which evaluates the
// exponent in the reference's order: for nearly singular conics (the
// highly anisotropic Gaussians of a stress scene) the terms cancel by four
// or more orders of magnitude and only the same rounding sequence
// reproduces the reference's alpha.
__device__ __forceinline__ bool conic_safe(float a, float b, float b2, float c) {
  return a > 0.0f && c > 0.0f && a * c - b * b2 > 0.02f * (a * c);
}

// Forward staged record: full quads only (a 12-byte LDS read occupies the
// LDS longer than a 16-byte one), and no list position (the loop tracks
// the batch-local index instead):
//   quad 0: (mx, my, kc*i00, kc*(i01 + i10))
//   quad 1: (kc*i11, log2(o w), re0, im0)
//   quad 2: (re1, im1, re2, im2)            (C >= 2)
// with kc = -log2(e)/2.  Exact batches stage the conic unscaled, in the
// reference's layout, followed by the amplitude quads of the global record:
//   quad 0: (mx, my, i00, i10)
//   quad 1: (i01, log2(o w), i11, 0)
//   quads 2..: (re0, im0, re1, im1), (re2, im2, 0, 0)
__host__ __device__ constexpr int fwd_quads(int C) { return C == 1 ? 2 : 3; }
__host__ __device__ constexpr int fwd_quads_exact(int C) { return rec_quads(C); }

// Exact-batch member evaluation: the exponent in the reference's order
// (forward_splat.cu:222-225), power = -0.5 s with
// s = dx (i00 dx + i10 dy) + dy (i01 dx + i11 dy), each product and sum
// rounded on its own (the library is built without contraction), the
// "power > 0: skip" test as s < 0, then alpha from exp2(kc s + log2(o w))
// (kc = -log2(e)/2, one rounding in the fused multiply-add).  The rest is
// fwd_member with the power test and the list index of the last
// contributor (`lastj` becomes j where the lane composites it; `real`
// (scalar) is false for padding members).
template <int C>
__device__ __forceinline__ void fwd_member_ref(const float4 a, const float4 b, const float4 c,
                                               const float4 d, float pxf, float pyf, float& T,
                                               float (&acc)[2 * C], int& lastj, int j,
                                               bool real) {
  const float dx = a.x - pxf, dy = a.y - pyf;
  const float s = dx * (a.z * dx + a.w * dy) + dy * (b.x * dx + b.z * dy);
  const bool live = !(T < kTermT);
  const bool ok = live && !(s < 0.0f);
  const float pw = fmaf(kBwdConicScale, s, b.y);
  const float alpha = ok ? fminf(kMaxAlpha, __builtin_amdgcn_exp2f(pw)) : 0.0f;
  const float sT = alpha * T;
  const float amp[6] = {c.x, c.y, c.z, c.w, d.x, d.y};
#pragma unroll
  for (int k = 0; k < C; ++k) {
    acc[2 * k] = fmaf(sT, amp[2 * k], acc[2 * k]);
    acc[2 * k + 1] = fmaf(sT, amp[2 * k + 1], acc[2 * k + 1]);
  }
  T = T * (1.0f - alpha);
  lastj = (ok && real) ? j : lastj;
}

// kTag: the list has pair tags (p.ptag): untagged entries are culled in
// every plane, so they are skipped without loading their plane mask or
// record; a block that ends with a pixel still live then looks for the
// last culled member among them from the list's end (for n_contrib).
template <int C, bool kTag>
__device__ __forceinline__ void render_fwd_block(const RenderParams& p) {
  constexpr int NQ = fwd_quads(C);
  constexpr int NQX = fwd_quads_exact(C);
  constexpr int RS = rec_stride(C);
  constexpr int kUnroll = 8;
  __shared__ float4 s_rec[kBlock * NQX];
  __shared__ int s_pos[kBlock];  // list position + 1 of each staged member
  __shared__ int s_wt[kBlock / 64];
  __shared__ int s_kcull;  // 1 + the largest list position culled as invisible

  int tile, plane;
  if (p.tile_order) {
    // Tiles longest list first; hardware block b runs on XCD b % 8, and in
    // each group of 8 P consecutive blocks XCD x takes the P planes of the
    // group's x-th tile (a tile's planes share its list in one L2).  The
    // last, partial group is taken in plain order.
    const int b = blockIdx.x, P = p.P, nt = p.tile_order_n;
    const int full = (nt / 8) * 8 * P;
    int rank;
    if (b < full) {
      const int grp = b / (8 * P), r = b - grp * 8 * P;
      rank = grp * 8 + (r & 7);
      plane = r >> 3;
    } else {
      const int r = b - full;
      rank = (nt / 8) * 8 + r / P;
      plane = r - (r / P) * P;
    }
    tile = p.tile_order[rank];
  } else {
    map_block(blockIdx.x, gridDim.x, p.P, &tile, &plane);
  }
  const int tx = tile % p.gx, ty = tile / p.gx;
  const int pxi = tx * kTile + (threadIdx.x & 15);
  const int pyi = ty * kTile + (threadIdx.x >> 4);
  const bool inside = pxi < p.W && pyi < p.H;
  int r0, n;
  tile_range(p, tile, &r0, &n);
  if (p.ranges_out && plane == 0 && threadIdx.x < 2)
    p.ranges_out[2 * tile + threadIdx.x] = p.ranges[2 * tile + threadIdx.x];
  // The pixel's offset from the tile centre (exact: small half-integers).
  const float xc = static_cast<float>(tx * kTile) + 0.5f * (kTile - 1);
  const float yc = static_cast<float>(ty * kTile) + 0.5f * (kTile - 1);
  const float u = static_cast<float>(pxi) - xc, v = static_cast<float>(pyi) - yc;

  // Lanes outside the image start done (T = 0 < 1e-4) and write nothing.
  float T = inside ? 1.0f : 0.0f;
  float acc[2 * C];
#pragma unroll
  for (int i = 0; i < 2 * C; ++i) acc[i] = 0.0f;
  int last = 0;
  int listed = 0;  // plane members of the batches composited so far
  int2* const sub_out =
      p.sub_out ? p.sub_out + static_cast<int64_t>(plane) * p.num_pairs + r0 : nullptr;

  const float tx0 = static_cast<float>(tx * kTile), ty0 = static_cast<float>(ty * kTile);
  if (threadIdx.x == 0) s_kcull = 0;
  // Each batch's list entries and their plane masks are loaded during the
  // previous batch: they depend only on the list, and two dependent loads
  // per batch (entry, then mask) would otherwise precede the record loads.
  int g_next = 0;
  uint32_t m_next = 0;
  if (!kTag && static_cast<int>(threadIdx.x) < n) {
    g_next = p.plist[r0 + static_cast<int>(threadIdx.x)];
    if (static_cast<uint64_t>(static_cast<uint32_t>(g_next)) < static_cast<uint64_t>(p.n))
      m_next = p.pmask[g_next];
  }
  __syncthreads();  // s_kcull's initialisation before the batches' culls
  // One batch: this thread's entry (list position k, gaussian g; mem: a
  // member of this plane) is culled, the block's members are staged and
  // composited.  Returns true, having staged nothing, once every pixel of
  // the block is done.  load_next / mask_next: the untagged walk's loads of
  // the next batch's entries and plane masks, issued before and after the
  // record loads.
  auto batch = [&](const int k, const int g, bool mem, auto&& load_next,
                   auto&& mask_next) -> bool {
    // geometry quads; the amplitude quads load at the LDS write
    float4 rq[2] = {make_float4(0.0f, 0.0f, 0.0f, 0.0f), make_float4(0.0f, 0.0f, 0.0f, 0.0f)};
    float w = 0.0f;
    unsigned qm4 = 0;  // quadrants the member reaches at alpha >= 1/255
    const float4* src = nullptr;
    load_next();
    if (mem) {
      src = reinterpret_cast<const float4*>(p.rec + static_cast<int64_t>(g) * RS);
      rq[0] = src[0];
      rq[1] = src[1];
      w = p.pprobs[static_cast<int64_t>(g) * p.P + plane];
      const float thr = invisible_threshold(rq[1].z * w);
      const CullShape cs = cull_shape(rq[0].z, rq[0].w, rq[1].y);
      if (!box_reaches(rq[0].x, rq[0].y, cs, thr, tx0, ty0, static_cast<float>(kTile - 1))) {
        mem = false;
        atomicMax(&s_kcull, k + 1);
      } else if (sub_out) {
        // The backward's per-quadrant alpha >= 1/255 test, with the same
        // threshold and shape (k_render_bwd's cull), for the list entry.
        const float thb = alpha_threshold(rq[1].z * w);
        if (thb >= 0.0f) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            qm4 |= box_reaches(rq[0].x, rq[0].y, cs, thb, tx0 + (q & 1) * 8, ty0 + (q >> 1) * 8,
                               7.0f)
                       ? (1u << q)
                       : 0u;
        }
      }
    }
    mask_next();
    // One barrier publishes each wave's member count (the compaction), whether
    // it stages a conic that is not safe (then the batch runs the exact
    // loop) and whether all its pixels are done (then the block is).  The
    // previous batch's LDS reads all precede it: its member loop ends before
    // the lanes reach this point.
    int pos, cnt = 0, spos = 0, scnt = 0;
    bool exact = false, clamp = false;
    {
      const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
      const uint64_t bal = __ballot(mem);
      const uint64_t bsub = __ballot(qm4 != 0u);
      const bool w_unsafe = __ballot(mem && !conic_safe(rq[0].z, rq[0].w, rq[1].x, rq[1].y)) != 0ull;
      const bool w_clamp = __ballot(mem && !(rq[1].z * w <= kNoClampOw)) != 0ull;
      const bool w_done = __ballot(!(T < kTermT)) == 0ull;
      if (lane == 0)
        s_wt[wave] = __popcll(bal) | (w_unsafe ? kWtUnsafe : 0) | (w_done ? kWtDone : 0) |
                     (w_clamp ? kWtClamp : 0) |
                     (__popcll(bsub) << kWtSubShift);
      __syncthreads();
      int off = 0, soff = 0;
      bool all_done = true;
#pragma unroll
      for (int wv = 0; wv < kBlock / 64; ++wv) {
        const int t = s_wt[wv];
        const int c = t & kWtCount;
        const int sc = (t >> kWtSubShift) & kWtCount;
        off += (wv < wave) ? c : 0;
        cnt += c;
        soff += (wv < wave) ? sc : 0;
        scnt += sc;
        exact = exact || (t & kWtUnsafe) != 0;
        clamp = clamp || (t & kWtClamp) != 0;
        all_done = all_done && (t & kWtDone) != 0;
      }
      if (all_done) return true;
      pos = off + bits_below_lane(bal);
      spos = soff + bits_below_lane(bsub);
    }
    if (mem) {
      if (qm4 != 0u)
        sub_out[listed + spos] = make_int2(g, static_cast<int>(static_cast<uint32_t>(k) |
                                                                (qm4 << kSubPosBits)));
      const float4 am = src[2];  // (re0, im0, re1, im1)
      const float lw = __builtin_amdgcn_logf(rq[1].z * w);
      if (!exact) {
        // The exponent as a quadratic in the offset from the tile centre
        // (fwd_member, quad_coeffs) for the scaled conic
        // (A, B, C) = kc (i00, i01 + i10, i11); c3..c5 = A, B, C.
        const float qa = kBwdConicScale * rq[0].z, qb = kBwdConicScale * (rq[0].w + rq[1].x);
        const float qc = kBwdConicScale * rq[1].y;
        float c0, c1, c2;
        quad_coeffs(rq[0].x, rq[0].y, qa, qb, qc, lw, xc, yc, &c0, &c1, &c2);
        s_rec[pos * NQ] = make_float4(c0, c1, c2, qa);
        s_rec[pos * NQ + 1] = make_float4(qb, qc, am.x, am.y);
        if (NQ > 2) {
          const float4 am2 = rec_quads(C) > 3 ? src[3] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          s_rec[pos * NQ + (NQ > 2 ? 2 : 0)] = make_float4(am.z, am.w, am2.x, am2.y);
        }
      } else {
        s_rec[pos * NQX] = make_float4(rq[0].x, rq[0].y, rq[0].z, rq[1].x);
        s_rec[pos * NQX + 1] = make_float4(rq[0].w, lw, rq[1].y, 0.0f);
        s_rec[pos * NQX + 2] = am;
        if (NQX > 3) s_rec[pos * NQX + (NQX > 3 ? 3 : 2)] = src[3];
      }
      s_pos[pos] = k + 1;
    }
    // Pad the staged batch to a multiple of kUnroll with members no pixel
    // can use: an exponent of -inf (alpha 0, T unchanged); in the exact
    // layout log2(o w) = -inf with a zero conic (s = 0, which passes the
    // power test).
    listed += scnt;
    const int cnt_pad = (cnt + kUnroll - 1) / kUnroll * kUnroll;
    if (static_cast<int>(threadIdx.x) >= cnt && static_cast<int>(threadIdx.x) < cnt_pad) {
      const int nq = exact ? NQX : NQ;
      const int q0 = static_cast<int>(threadIdx.x) * nq;
      // Materialised here: hoisted out of the batch loop, these constants
      // would not fit the 64 registers of 8 waves per SIMD.
      float far = 1e6f, ninf = -__builtin_inff(), zero = 0.0f;
      asm volatile("" : "+v"(far), "+v"(ninf), "+v"(zero));
      if (!exact) {
        // c0 = -inf, the other coefficients 0: pw = -inf at every pixel
        s_rec[q0] = make_float4(ninf, zero, zero, zero);
        s_rec[q0 + 1] = make_float4(zero, zero, zero, zero);
      } else {
        s_rec[q0] = make_float4(far, far, zero, zero);
        s_rec[q0 + 1] = make_float4(zero, ninf, zero, zero);
      }
#pragma unroll
      for (int q = 2; q < NQX; ++q)
        if (q < nq) s_rec[q0 + q] = make_float4(zero, zero, zero, zero);
    }
    __syncthreads();
    // Branch-free per member; a wave leaves the batch once all its lanes
    // are done.
    const bool live0 = !(T < kTermT);
    int lastj = -1;
    if (!exact) {
      // Instantiated with and without the alpha clamp (kNoClampOw).
      auto fast = [&](auto clamp_tag) {
        constexpr bool kClamp = decltype(clamp_tag)::value;
        int evaluated = 0;
        for (int j0 = 0; j0 < cnt_pad; j0 += kUnroll) {
          if (__all(T < kTermT)) break;
#pragma unroll
          for (int jj = 0; jj < kUnroll; ++jj) {
            const int j = j0 + jj;
            fwd_member<C, kClamp>(s_rec[j * NQ], s_rec[j * NQ + 1], s_rec[j * NQ + (NQ - 1)], u,
                                  v, T, acc, evaluated);
          }
        }
        // A lane still running composited every member of the batch (no
        // power test could fail): the batch's last member is its last
        // contributor.  One that terminated here composited members
        // 0..evaluated-1 (padding follows every real member, so it ended on
        // a real one).
        lastj = !(T < kTermT) ? cnt - 1 : evaluated - 1;
      };
      if (clamp)
        fast(std::true_type{});
      else
        fast(std::false_type{});
    } else {
      for (int j0 = 0; j0 < cnt_pad; j0 += kUnroll) {
        if (__all(T < kTermT)) break;
        // four at a time: the unscaled layout's fourth quad would not fit
        // the 64 registers of 8 waves per SIMD at eight
#pragma unroll 2
        for (int jj = 0; jj < kUnroll; ++jj) {
          const int j = j0 + jj;
          fwd_member_ref<C>(s_rec[j * NQX], s_rec[j * NQX + 1], s_rec[j * NQX + 2],
                            s_rec[j * NQX + (NQX - 1)], u + xc, v + yc, T, acc, lastj, j,
                            j < cnt);
        }
      }
    }
    if (live0 && lastj >= 0) last = s_pos[lastj];
    return false;
  };

  if constexpr (!kTag) {
    for (int base = 0; base < n; base += kBlock) {
      const int k = base + static_cast<int>(threadIdx.x);
      const int g = g_next;
      const bool mem = k < n &&
                       static_cast<uint64_t>(static_cast<uint32_t>(g)) < static_cast<uint64_t>(p.n) &&
                       ((m_next >> plane) & 1u);
      const bool done = batch(
          k, g, mem,
          [&] {
            const int kn = k + kBlock;
            g_next = kn < n ? p.plist[r0 + kn] : 0;
            m_next = 0;
          },
          [&] {
            if (k + kBlock < n &&
                static_cast<uint64_t>(static_cast<uint32_t>(g_next)) < static_cast<uint64_t>(p.n))
              m_next = p.pmask[g_next];
          });
      if (done) break;
    }
  } else {
    // Tagged lists: windows of kTagWin entries; the tagged positions of a
    // window (tag bytes only, in list order) are compacted into s_cand and
    // staged in batches of kBlock, so a block walks its list in a fraction
    // of the batches (config 4 tags ~5% of its entries).  Candidate order:
    // (i, wave, lane) for entry wb + i kBlock + threadIdx.x, which is list
    // order.
    constexpr int kPer = kTagWin / kBlock;
    __shared__ unsigned short s_cand[kTagWin];
    __shared__ int s_wc[kBlock / 64][kPer];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int wb = 0; wb < n; wb += kTagWin) {
      uint64_t bal[kPer];
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int k = wb + i * kBlock + static_cast<int>(threadIdx.x);
        bal[i] = __ballot(k < n && p.ptag[r0 + k] != 0);
      }
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) s_wc[wave][i] = __popcll(bal[i]);
      }
      // (the block leaves once every pixel is done)
      if (!__syncthreads_or(!(T < kTermT))) break;
      int ncand = 0;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        int off = ncand;
#pragma unroll
        for (int wv = 0; wv < kBlock / 64; ++wv) {
          const int c = s_wc[wv][i];
          off += (wv < wave) ? c : 0;
          ncand += c;
        }
        if ((bal[i] >> lane) & 1ull)
          s_cand[off + bits_below_lane(bal[i])] =
              static_cast<unsigned short>(i * kBlock + static_cast<int>(threadIdx.x));
      }
      __syncthreads();
      bool done = false;
      for (int cb = 0; cb < ncand; cb += kBlock) {
        const int ci = cb + static_cast<int>(threadIdx.x);
        int k = 0, g = -1;
        uint32_t m = 0;
        if (ci < ncand) {
          k = wb + static_cast<int>(s_cand[ci]);
          g = p.plist[r0 + k];
          if (static_cast<uint64_t>(static_cast<uint32_t>(g)) < static_cast<uint64_t>(p.n))
            m = p.pmask[g];
        }
        const bool mem = ci < ncand && ((m >> plane) & 1u);
        if (batch(k, g, mem, [] {}, [] {})) {
          done = true;
          break;
        }
      }
      if (done) break;
    }
  }

  if (kTag && __syncthreads_or(!(T < kTermT))) {
    // Some pixel composited the whole list, the skipped (untagged) members
    // of this plane included: the last of them, if past s_kcull, is its
    // last contributor.  Scanned from the list's end, one batch at a time,
    // until a batch holds one.
    for (int top = n; top > 0; top -= kBlock) {
      const int k = top - 1 - static_cast<int>(threadIdx.x);
      bool cand = false;
      if (k >= 0 && p.ptag[r0 + k] == 0) {
        const int g = p.plist[r0 + k];
        cand = static_cast<uint64_t>(static_cast<uint32_t>(g)) < static_cast<uint64_t>(p.n) &&
               ((p.pmask[g] >> plane) & 1u);
      }
      if (cand) atomicMax(&s_kcull, k + 1);
      if (__syncthreads_or(cand)) break;
    }
  }
  if (sub_out && threadIdx.x == 0) p.sub_cnt_out[tile * p.P + plane] = listed;
  __syncthreads();
  // A pixel that never terminated composited every member, culled ones too.
  if (!(T < kTermT)) last = max(last, s_kcull);
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
__global__ __launch_bounds__(kBlock, C == 2 ? 7 : 8) void k_render_fwd(RenderParams p) {
  render_fwd_block<C, false>(p);
}
template <int C>
__global__ __launch_bounds__(kBlock, C == 2 ? 7 : 8) void k_render_fwd_tagged(RenderParams p) {
  render_fwd_block<C, true>(p);
}

// Backward staged record: the global record's quad count, one more at C = 2
// for 1/det (see k_render_bwd).
__host__ __device__ constexpr int bwd_quads(int C) { return C == 2 ? 4 : rec_quads(C); }

// 1/det of the staged member's cov2D from its amplitude quads (c0 = quad 2,
// c1 = the last quad).
template <int C>
__device__ __forceinline__ float bwd_det_inv(const float4 c0, const float4 c1) {
  return C == 1 ? c0.z : (C == 2 ? c1.x : c1.z);
}

// Backward.  Waves own 8x8 quadrants of the tile.  Per batch, every staged
// Gaussian gets a 4-bit quadrant mask (its alpha >= 1/255 region meets the
// quadrant and its list position is below that quadrant's max n_contrib);
// each wave walks only its own compacted list, back to front, in groups of
// G members whose 6+2C partial sums per lane are reduced together with one
// transpose_reduce64.  Skipping a member for a whole wave is exact: every
// lane of that wave would skip it (alpha < 1/255 or position >= n_contrib).
template <int C, bool kSub>
__global__ __launch_bounds__(kBlock, C == 3 ? (kSub ? 5 : 4) : 2) void k_render_bwd(RenderParams p) {
  // Staged record: quads 0-1 as below, then the amplitude quads of the
  // global record, with 1/det of the member's cov2D in the first free slot
  // after the amplitudes (an extra quad at C = 2).  Fast batches: quad 0
  // (mx, my, kc cxx, 2 kc cxy), quad 1 (kc czz, log2(o w), k, o w).  Exact
  // batches stage the conic unscaled, in the reference's backward form:
  // quad 0 (mx, my, cxx, cxy), quad 1 (czz, log2(o w), k, o w).
  constexpr int NQ = bwd_quads(C);
  constexpr int RS = rec_stride(C);
  constexpr int NV = 6 + 2 * C;  // partial sums per member
  constexpr int NVP = (NV + 3) / 4 * 4;  // padded for row_sum16
  static_assert(NVP <= 16, "one 16-lane row holds a member's sums");
  constexpr int G = kBwdChunk;
  // A batch stages kStage = 255 list entries, so that a slot index fits a
  // byte (the per-wave lists are bytes and the Gaussian index rides in the
  // staged record's last word: 32 KB of LDS, 5 blocks per CU).  Slot kStage
  // of s_rec is a dummy member that no pixel can use (list position beyond
  // every n_contrib): the per-wave lists are padded with it to a multiple
  // of G, so the member loop needs no bounds.  It is written per batch.
  constexpr int kStage = kBlock - 1;
  constexpr int kDummy = kStage;
  __shared__ float4 s_rec[(kStage + 1) * NQ];
  __shared__ unsigned char s_wl[4][kBlock + G];
  __shared__ int s_cnt[4][5];
  __shared__ int s_wmax[4];
  // Per wave: the chunk's (Q, dcol) per (member, pixel), written by the
  // pixel lanes and read by the member lanes; the quadrant's upstream
  // gradient per pixel (re, im per channel).
  __shared__ float2 s_qd[4][G][64];
  __shared__ float2 s_gp[4][64][C];

  int tile, plane;
  if (kSub) {
    // Longest member list first (list scheduling): the forward's per-(tile,
    // plane) member counts order the blocks.
    const int id = p.order[blockIdx.x];
    if (static_cast<unsigned>(id) >= gridDim.x) return;
    tile = id / p.P;
    plane = id - tile * p.P;
  } else {
    map_block(blockIdx.x, gridDim.x, p.P, &tile, &plane);
  }
  const int tx = tile % p.gx, ty = tile / p.gx;
  // wave is the same in every lane; read it as a scalar so that what is
  // derived from it (and from the per-wave LDS counts below) stays scalar.
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int pxi = tx * kTile + (wave & 1) * 8 + (lane & 7);
  const int pyi = ty * kTile + (wave >> 1) * 8 + (lane >> 3);
  const bool inside = pxi < p.W && pyi < p.H;
  int r0, n;
  tile_range(p, tile, &r0, &n);
  const float pxf = static_cast<float>(pxi), pyf = static_cast<float>(pyi);
  const int64_t HW = static_cast<int64_t>(p.W) * p.H;
  const int64_t pix = static_cast<int64_t>(pyi) * p.W + pxi;
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
#pragma unroll
  for (int c = 0; c < C; ++c) s_gp[wave][lane][c] = make_float2(gre[c], gim[c]);
  {
    int m = inside ? last : 0;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) m = max(m, __shfl_xor(m, d, 64));
    if (lane == 0) s_wmax[wave] = m < n ? m : n;
  }
  __syncthreads();
  int wmax[4];
  int maxlast = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    wmax[w] = s_wmax[w];
    maxlast = max(maxlast, wmax[w]);
  }

  float R = 0.0f, pend = 0.0f;
  const float half_w = 0.5f * static_cast<float>(p.W);
  const float half_h = 0.5f * static_cast<float>(p.H);
  const float tx0 = static_cast<float>(tx * kTile), ty0 = static_cast<float>(ty * kTile);
  const float qx0 = tx0 + static_cast<float>((wave & 1) * 8);  // this wave's quadrant
  const float qy0 = ty0 + static_cast<float>((wave >> 1) * 8);

  // Entries walked: list positions [0, maxlast) of the tile list, or the
  // whole member list of this plane (entries at positions >= maxlast are
  // then culled by the quadrant bounds below).
  int lim = maxlast;
  const int2* sub = nullptr;
  if (kSub) {
    const int c = p.sub_cnt[tile * p.P + plane];
    lim = c < 0 ? 0 : (c > n ? n : c);
    sub = p.sub + static_cast<int64_t>(plane) * p.num_pairs + r0;
  }
  for (int end = lim; end > 0; end -= kStage) {
    const int start = end > kStage ? end - kStage : 0;
    // No barrier here: until the count barrier below, a batch writes only
    // s_cnt, which the previous batch last read before its member loop; the
    // staging writes that the previous flush's reads must precede come after
    // that barrier.
    const int idx = start + static_cast<int>(threadIdx.x);
    int k = idx;
    int g = 0;
    unsigned qm = 0;
    bool ill = false;  // conic outside the fast loop's domain (conic_safe)
    float4 rq[2];  // quads 0-1 (geometry); the amplitude quads load once culled
    float wpl = 0.0f;
    const float4* src = nullptr;
    if (idx < end && kSub) {
      // The forward's quadrant mask (alpha >= 1/255 box test); only the
      // n_contrib bounds remain, and only survivors gather their records.
      const int2 e = sub[idx];
      g = e.x;
      k = static_cast<int>(static_cast<uint32_t>(e.y) & kSubPosMask);
      const uint32_t m4 = static_cast<uint32_t>(e.y) >> kSubPosBits;
#pragma unroll
      for (int w = 0; w < 4; ++w) qm |= (((m4 >> w) & 1u) && k < wmax[w]) ? (1u << w) : 0u;
      if (static_cast<uint64_t>(static_cast<uint32_t>(g)) >= static_cast<uint64_t>(p.n)) qm = 0;
      if (qm != 0u) {
        src = reinterpret_cast<const float4*>(p.rec + static_cast<int64_t>(g) * RS);
        rq[0] = src[0];
        rq[1] = src[1];
        wpl = p.pprobs[static_cast<int64_t>(g) * p.P + plane];
        ill = !conic_safe(rq[0].z, rq[0].w, rq[0].w, rq[1].y);
      }
    } else if (idx < end) {
      g = p.plist[r0 + idx];
      const bool member =
          static_cast<uint64_t>(static_cast<uint32_t>(g)) < static_cast<uint64_t>(p.n) &&
          ((p.pmask[g] >> plane) & 1u);
      if (member) {
        src = reinterpret_cast<const float4*>(p.rec + static_cast<int64_t>(g) * RS);
        rq[0] = src[0];
        rq[1] = src[1];
        wpl = p.pprobs[static_cast<int64_t>(g) * p.P + plane];
        const float thr = alpha_threshold(rq[1].z * wpl);
        if (thr >= 0.0f) {
          ill = !conic_safe(rq[0].z, rq[0].w, rq[0].w, rq[1].y);
          const CullShape cs = cull_shape(rq[0].z, rq[0].w, rq[1].y);
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float x0 = tx0 + (w & 1) * 8, y0 = ty0 + (w >> 1) * 8;
            const bool hit = k < wmax[w] && box_reaches(rq[0].x, rq[0].y, cs, thr, x0, y0, 7.0f);
            qm |= hit ? (1u << w) : 0u;
          }
        }
      }
    }
    uint64_t bal[5];
    bal[0] = __ballot(qm != 0u);
#pragma unroll
    for (int w = 0; w < 4; ++w) bal[1 + w] = __ballot((qm >> w) & 1u);
    // A batch staging any conic outside the fast loop's domain runs the
    // reference-order loop (the flag rides in the wave's staged count).
    const bool w_ill = __ballot(qm != 0u && ill) != 0ull;
    // ... and one staging a member with o w above kNoClampOw keeps the alpha
    // clamp.
    const bool w_clamp = __ballot(qm != 0u && !(rq[1].z * wpl <= kNoClampOw)) != 0ull;
    if (lane == 0) {
#pragma unroll
      for (int f = 0; f < 5; ++f)
        s_cnt[wave][f] = __popcll(bal[f]) | (f == 0 && w_ill ? 0x100 : 0) |
                         (f == 0 && w_clamp ? 0x200 : 0);
    }
    __syncthreads();
    int off[5], tot[5];
    bool exact = false, clamp = false;
#pragma unroll
    for (int f = 0; f < 5; ++f) {
      off[f] = 0;
      tot[f] = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int sc = __builtin_amdgcn_readfirstlane(s_cnt[w][f]);  // same in every lane
        const int c = sc & 0xFF;
        if (f == 0) exact = exact || (sc & 0x100) != 0;
        if (f == 0) clamp = clamp || (sc & 0x200) != 0;
        off[f] += (w < wave) ? c : 0;
        tot[f] += c;
      }
      off[f] += bits_below_lane(bal[f]);
    }
    const int cnt = tot[0];
    if (static_cast<int>(threadIdx.x) < NQ)
      s_rec[kDummy * NQ + threadIdx.x] =
          threadIdx.x == 0   ? make_float4(1e6f, 1e6f, 0.0f, 0.0f)
          : threadIdx.x == 1 ? make_float4(0.0f, 0.0f, __int_as_float(0x7FFFFFFF), 1.0f)
                             : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (qm != 0u) {
      const int slot = off[0];
      // quad 0: (mx, my, kc*cxx, 2 kc*cxy); quad 1: (kc*czz, log2(o*w), k,
      // o*w) with kc = -log2(e)/2, so pw = dx (kc cxx dx + 2 kc cxy dy) +
      // kc czz dy^2 + log2(o w) is log2(e) * power + log2(o w) and
      // exp2(pw) = o w G (the reference's backward exponent: one
      // off-diagonal, doubled, backward_splat.cu:208-210).  Quad 1 also
      // carries the list position (int bits) for the n_contrib test.
      // Amplitude quads only for members that survived the cull (same
      // 64-byte record as quads 0-1, so the loads hit the cache).
      const float ow = rq[1].z * wpl;
      const float lw = __builtin_amdgcn_logf(ow);
      if (!exact) {
        s_rec[slot * NQ] = make_float4(rq[0].x, rq[0].y, kBwdConicScale * rq[0].z,
                                       2.0f * kBwdConicScale * rq[0].w);
        s_rec[slot * NQ + 1] = make_float4(kBwdConicScale * rq[1].y, lw, __int_as_float(k), ow);
      } else {
        s_rec[slot * NQ] = rq[0];
        s_rec[slot * NQ + 1] = make_float4(rq[1].y, lw, __int_as_float(k), ow);
      }
      const float4 am0 = src[2];
      const float4 am1 = rec_quads(C) > 3 ? src[rec_quads(C) > 3 ? 3 : 2] : am0;
      // The last quad's last word: the Gaussian index (int bits).
      const float gb = __int_as_float(g);
      if (C == 1) {
        s_rec[slot * NQ + 2] = make_float4(am0.x, am0.y, rq[1].w, gb);
      } else if (C == 2) {
        s_rec[slot * NQ + 2] = am0;
        s_rec[slot * NQ + (NQ > 3 ? 3 : 2)] = make_float4(rq[1].w, 0.0f, 0.0f, gb);
      } else {
        s_rec[slot * NQ + 2] = am0;
        s_rec[slot * NQ + (NQ > 3 ? 3 : 2)] = make_float4(am1.x, am1.y, rq[1].w, gb);
      }
      // Each wave's list is stored after its padding, so it ends at a
      // multiple of G.
#pragma unroll
      for (int w = 0; w < 4; ++w)
        if ((qm >> w) & 1u)
          s_wl[w][(G - tot[1 + w] % G) % G + off[1 + w]] = static_cast<unsigned char>(slot);
    }
    if (static_cast<int>(threadIdx.x) < 4 * G) {
      const int w = threadIdx.x / G, j = threadIdx.x - w * G;
      // tot[1 + w] by selects: a runtime index would put tot[] in scratch
      const int tw = w == 0 ? tot[1] : (w == 1 ? tot[2] : (w == 2 ? tot[3] : tot[4]));
      if (j < (G - tw % G) % G) s_wl[w][j] = static_cast<unsigned char>(kDummy);
    }
    __syncthreads();

    int nl = 0;  // this wave's padded list length (a multiple of G)
#pragma unroll
    for (int w = 0; w < 4; ++w) nl = (w == wave) ? tot[1 + w] + (G - tot[1 + w] % G) % G : nl;
    // The member walk in chunks of G members, back to front, instantiated
    // for the fast exponent and for the reference-order one (exact batches).
    auto walk = [&](auto ref_tag, auto clamp_tag) {
      constexpr bool kRef = decltype(ref_tag)::value;
      constexpr bool kClamp = decltype(clamp_tag)::value;
      for (int hi = nl - 1; hi >= 0; hi -= G) {
        // Phase 1, one pixel per lane: the back-to-front recurrence over the
        // chunk's members, branch-free (a member that does not contribute at
        // the pixel takes G = alpha = 0: T / 1 and 0 * x leave T and the
        // sums exactly unchanged), leaving per (member, pixel) Q = o w G
        // dL/dG and dcol = alpha T in LDS.
        bool any = false;
#pragma unroll
        for (int m = 0; m < G; ++m) {
          const int slot = s_wl[wave][hi - m];
          const float4 a = s_rec[slot * NQ];
          const float4 b = s_rec[slot * NQ + 1];
          const int kk = __float_as_int(b.z);
          const float dx = a.x - pxf, dy = a.y - pyf;
          bool ok;
          float Ga;  // o w G
          if (kRef) {
            // backward_splat.cu:211 in its order, each step rounded on its own
            const float power = -0.5f * (a.z * dx * dx + b.x * dy * dy) - a.w * dx * dy;
            Ga = __builtin_amdgcn_exp2f(fmaf(kLog2E, power, b.y));
            ok = kk < last && !(power > 0.0f) && fminf(kMaxAlpha, Ga) >= kMinAlphaBwd;
          } else {
            // A conic in this loop's domain cannot round to a positive
            // exponent, and its alpha is finite: the alpha test reads o w G.
            const float t = fmaf(a.z, dx, a.w * dy);
            Ga = __builtin_amdgcn_exp2f(fmaf(dx, t, fmaf(b.x * dy, dy, b.y)));
            ok = kk < last && Ga >= kMinAlphaBwd;
          }
          any = any || ok;
          const float Gz = ok ? Ga : 0.0f;
          const float ae = kClamp ? fminf(kMaxAlpha, Gz) : Gz;
          T = div_rn(T, 1.0f - ae);
          const float dcol = ae * T;
          // Re(colour * conj(g)) summed over channels; the reference's
          // complex recurrence acc = la*last + (1-la)*acc is linear, so only
          // its projection R = sum_c Re(acc_c conj(g_c)) is carried.
          const float4 c0 = s_rec[slot * NQ + 2];
          const float4 c1 = s_rec[slot * NQ + (NQ > 3 ? 3 : 2)];
          const float amp[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
          float S = amp[0] * gre[0];
          S = fmaf(amp[1], gim[0], S);
#pragma unroll
          for (int c = 1; c < C; ++c) {
            S = fmaf(amp[2 * c], gre[c], S);
            S = fmaf(amp[2 * c + 1], gim[c], S);
          }
          // acc = a_l S_l + (1 - a_l) acc over the contributing members: R
          // advances by the pending a_l (S_l - R) of the previous
          // contributor, and this member's becomes pending.  A
          // non-contributor (alpha 0) takes the pending increment early and
          // leaves none, so the updates need no selects.
          R += pend;
          const float dS = S - R;
          pend = ae * dS;
          s_qd[wave][m][lane] = make_float2(Gz * (dS * T), dcol);
        }
        if (__ballot(any) == 0ull) continue;
        // The pixel lanes' writes before the member lanes' reads (one wave:
        // the LDS keeps its order; this keeps the compiler's).
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // Phase 2, lane (member mm = lane / 16, part sp = lane % 16): the
        // member's NV partial sums over 4 pixels of the quadrant (column
        // sp % 8, rows sp / 8 + 2j), in registers; then the 16 lanes of the
        // member's row reduce them (row_sum16: each lane ends with NVP/4 of
        // the sums) and each lane with a sum to add adds it to the member's
        // accumulator.
        const int mm = lane >> 4, sp = lane & 15;
        const int slot2 = s_wl[wave][hi - mm];
        const float4 a2 = s_rec[slot2 * NQ];
        const float4 b2 = s_rec[slot2 * NQ + 1];
        const float4 c02 = s_rec[slot2 * NQ + 2];
        const float4 c12 = s_rec[slot2 * NQ + (NQ > 3 ? 3 : 2)];
        const float di2 = bwd_det_inv<C>(c02, c12);
        const int col = sp & 7;
        const float dx = a2.x - (qx0 + static_cast<float>(col));
        float v[NVP];
#pragma unroll
        for (int i = 0; i < NVP; ++i) v[i] = 0.0f;
        float Qj[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = (sp >> 3) + 2 * j;
          const int pp = row * 8 + col;
          const float2 qd = s_qd[wave][mm][pp];
          const float Q = qd.x, dcol = qd.y;
          Qj[j] = Q;
          if (kRef) {
            // exact batches: the reference's conic-to-covariance map per
            // pixel (backward_splat.cu:285-291) with the unscaled conic: xx =
            // cxx^2 U + cxy^2 W, xy = cxx cxy U - V / det + cxy czz W, yy =
            // cxy^2 U + czz^2 W for the pixel's second moments (U, V, W) =
            // Q (dx^2, dx dy, dy^2), all terms of one sign, so no sum is
            // mapped afterwards (for a nearly singular conic the map would
            // amplify the sums' rounding by ~1/(1 - r^2)).
            const float dy = a2.y - (qy0 + static_cast<float>(row));
            const float Qdx = Q * dx, Qdy = Q * dy;
            const float u = Qdx * dx, vv = Qdx * dy, w = Qdy * dy;
            v[0] = fmaf(Q, fmaf(a2.z, dx, a2.w * dy), v[0]);
            v[1] = fmaf(Q, fmaf(a2.w, dx, b2.x * dy), v[1]);
            v[2] = fmaf(a2.z * a2.z, u, fmaf(a2.w * a2.w, w, v[2]));
            v[3] = fmaf(a2.z * a2.w, u, fmaf(-di2, vv, fmaf(a2.w * b2.x, w, v[3])));
            v[4] = fmaf(a2.w * a2.w, u, fmaf(b2.x * b2.x, w, v[4]));
            v[5] += Q;
          }
#pragma unroll
          for (int c = 0; c < C; ++c) {
            const float2 gv = s_gp[wave][pp][c];
            v[6 + c] = fmaf(dcol, gv.x, v[6 + c]);
            v[6 + C + c] = fmaf(dcol, gv.y, v[6 + C + c]);
          }
        }
        if (!kRef) {
          // The geometric sums from three moments of Q over the lane's rows:
          // with dyc = dy at the rows' centre, row j has dy = dyc - e_j, e_j
          // = 2j - 3 (exact small integers), so sum Q dy = dyc B0 - B1 and
          // sum Q dy^2 = dyc (dyc B0 - 2 B1) + B2 for B_k = sum e_j^k Q_j;
          // dx is the lane's own.
          const float dyc = a2.y - (qy0 + static_cast<float>((sp >> 3) + 3));
          const float s03 = Qj[0] + Qj[3], s12 = Qj[1] + Qj[2];
          const float d03 = Qj[3] - Qj[0], d12 = Qj[2] - Qj[1];
          const float B0 = s03 + s12;
          const float B1 = fmaf(3.0f, d03, d12);
          const float B2 = fmaf(9.0f, s03, s12);
          const float m = dyc * B0;
          const float sy = m - B1;                                // sum Q dy
          const float syy = fmaf(dyc, fmaf(-2.0f, B1, m), B2);  // sum Q dy^2
          const float sx = dx * B0;                               // sum Q dx
          // The mean and covariance maps on the lane's sums (linear in them;
          // the conic is in the fast loop's domain, so the maps are well
          // conditioned).  Staged conic: kc cxx, 2 kc cxy, kc czz.
          const float kxy = 0.5f * a2.w;
          v[0] = fmaf(a2.z, sx, kxy * sy);  // kc (cxx sum Q dx + cxy sum Q dy)
          v[1] = fmaf(kxy, sx, b2.x * sy);  // kc (cxy sum Q dx + czz sum Q dy)
          const float cxx = a2.z * (1.0f / kBwdConicScale);
          const float cxy = a2.w * (0.5f / kBwdConicScale);
          const float czz = b2.x * (1.0f / kBwdConicScale);
          const float U = dx * sx, V = dx * sy, Wm = syy;
          v[2] = fmaf(cxx * cxx, U, (cxy * cxy) * Wm);
          v[3] = fmaf(cxx * cxy, U, fmaf(-di2, V, (cxy * czz) * Wm));
          v[4] = fmaf(cxy * cxy, U, (czz * czz) * Wm);
          v[5] = B0;
        }
        float xs[NVP / 4];
        row_sum16<NVP>(v, xs);
        // This lane's sum: value vi of the member (row_sum16's layout).
        const int q = sp & 3;
        const int vi = (NVP / 2) * ((sp >> 3) & 1) + (NVP / 4) * ((sp >> 2) & 1) + q;
        float tv = xs[0];
#pragma unroll
        for (int i = 1; i < NVP / 4; ++i) tv = (q == i) ? xs[i] : tv;
        // Accumulator slots: 0-1 the mean gradient (times W/2, H/2), 2-4 the
        // cov2D gradient, 5+c / 5+C+c the colour sums, 5+2C+plane the plane
        // term.  The sums carry o w (Q = o w dL/dG): the mean and covariance
        // terms need exactly that factor, the o w term (sum G dL/dalpha) its
        // removal.  Slot and scale are fixed per lane except that removal
        // (selects, so that they stay out of the loop).
        const int aslot = vi == 5 ? 5 + 2 * C + plane : (vi < 5 ? vi : vi - 1);
        const float scale_mean = vi == 0 ? half_w : half_h;
        const float scale_l =
            vi < 2 ? (kRef ? -scale_mean : scale_mean * (-1.0f / kBwdConicScale))
                   : (vi < 5 ? -0.5f : 1.0f);
        const float scale = vi == 5 ? __builtin_amdgcn_rcpf(b2.w) : scale_l;
        if (q < NVP / 4 && vi < NV && slot2 != kDummy && tv != 0.0f)
          unsafeAtomicAdd(p.acc + static_cast<int64_t>(__float_as_int(c12.w)) * AS + aslot,
                          tv * scale);
        // The next chunk's phase-1 writes after this chunk's reads.
        __builtin_amdgcn_wave_barrier();
      }
    };
    if (exact)
      walk(std::true_type{}, std::true_type{});
    else if (clamp)
      walk(std::false_type{}, std::true_type{});
    else
      walk(std::false_type{}, std::false_type{});
  }
}

constexpr int kOrderThreads = 1024;
constexpr int kOrderBins = 256;

// order[0..m) = the ids sorted by cost bucket, highest first; one block of
// kOrderThreads threads.
__device__ __forceinline__ void order_by_cost_block(const int32_t* cnt, int m, int32_t* order) {
  __shared__ int s_bin[kOrderBins];
  for (int i = threadIdx.x; i < kOrderBins; i += kOrderThreads) s_bin[i] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < m; i += kOrderThreads) atomicAdd(&s_bin[cost_bucket(cnt[i])], 1);
  __syncthreads();
  if (threadIdx.x < 64) {
    // Exclusive scan over the bins from the highest bucket down: lane l owns
    // bins 255-4l .. 252-4l.
    const int lane = threadIdx.x;
    int v[4], sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = s_bin[kOrderBins - 1 - 4 * lane - j];
      sum += v[j];
    }
    int inc = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int t = __shfl_up(inc, d, 64);
      if (lane >= d) inc += t;
    }
    int run = inc - sum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s_bin[kOrderBins - 1 - 4 * lane - j] = run;
      run += v[j];
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < m; i += kOrderThreads) {
    const int pos = atomicAdd(&s_bin[cost_bucket(cnt[i])], 1);
    order[pos] = i;
  }
}

// Backward prologue: block 0 forms the backward's (tile, plane) block order
// from the forward's member counts (when `order` is given) while the other
// blocks clear the accumulator records (n4 float4s, then `tail` floats).
__global__ __launch_bounds__(kOrderThreads) void k_bwd_prologue(float4* __restrict__ acc4,
                                                                int64_t n4,
                                                                float* __restrict__ tail,
                                                                int ntail, const int32_t* cnt,
                                                                int m, int32_t* order) {
  if (blockIdx.x == 0) {
    if (order) order_by_cost_block(cnt, m, order);
    return;
  }
  const int64_t stride = static_cast<int64_t>(gridDim.x - 1) * kOrderThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x - 1) * kOrderThreads + threadIdx.x; i < n4;
       i += stride)
    acc4[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (blockIdx.x == 1 && static_cast<int>(threadIdx.x) < ntail) tail[threadIdx.x] = 0.0f;
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
  const bool tag = p.ptag != nullptr;
  switch (p.C) {
    case 1:
      if (tag) hipLaunchKernelGGL(k_render_fwd_tagged<1>, dim3(nblocks), dim3(kBlock), 0, s, p);
      else hipLaunchKernelGGL(k_render_fwd<1>, dim3(nblocks), dim3(kBlock), 0, s, p);
      break;
    case 2:
      if (tag) hipLaunchKernelGGL(k_render_fwd_tagged<2>, dim3(nblocks), dim3(kBlock), 0, s, p);
      else hipLaunchKernelGGL(k_render_fwd<2>, dim3(nblocks), dim3(kBlock), 0, s, p);
      break;
    case 3:
      if (tag) hipLaunchKernelGGL(k_render_fwd_tagged<3>, dim3(nblocks), dim3(kBlock), 0, s, p);
      else hipLaunchKernelGGL(k_render_fwd<3>, dim3(nblocks), dim3(kBlock), 0, s, p);
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
      if (p.sub) hipLaunchKernelGGL((k_render_bwd<1, true>), dim3(nblocks), dim3(kBlock), 0, s, p);
      else hipLaunchKernelGGL((k_render_bwd<1, false>), dim3(nblocks), dim3(kBlock), 0, s, p);
      break;
    case 2:
      if (p.sub) hipLaunchKernelGGL((k_render_bwd<2, true>), dim3(nblocks), dim3(kBlock), 0, s, p);
      else hipLaunchKernelGGL((k_render_bwd<2, false>), dim3(nblocks), dim3(kBlock), 0, s, p);
      break;
    case 3:
      if (p.sub) hipLaunchKernelGGL((k_render_bwd<3, true>), dim3(nblocks), dim3(kBlock), 0, s, p);
      else hipLaunchKernelGGL((k_render_bwd<3, false>), dim3(nblocks), dim3(kBlock), 0, s, p);
      break;
    default:
      set_error("render backward: channels must be 1..3 (got %d)", p.C);
      return HRF_ERR_INVALID;
  }
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_bwd_prologue(float* acc, int64_t n, const int32_t* cnt, int m, int32_t* order,
                        hipStream_t s) {
  if (reinterpret_cast<uintptr_t>(acc) & 15) {
    set_error("internal: accumulator records not 16-byte aligned");
    return HRF_ERR_INVALID;
  }
  const int64_t n4 = n / 4;
  const int ntail = static_cast<int>(n - 4 * n4);
  const int64_t per = static_cast<int64_t>(kOrderThreads) * 4;  // float4s per block
  int64_t fill_blocks = (n4 + per - 1) / per;
  if (fill_blocks < 1) fill_blocks = 1;
  hipLaunchKernelGGL(k_bwd_prologue, dim3(static_cast<unsigned>(1 + fill_blocks)),
                     dim3(kOrderThreads), 0, s, reinterpret_cast<float4*>(acc), n4,
                     acc + 4 * n4, ntail, cnt, m, (m > 0 ? order : nullptr));
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
