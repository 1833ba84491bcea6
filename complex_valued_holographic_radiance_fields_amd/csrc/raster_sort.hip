// raster_sort.hip — stage 2: device scans, the stable LSD radix sort, pair
// emission in depth-rank order and tile ranges.
//
// Binning order.  The reference emits (tile<<32 | depth') keys in Gaussian
// index order and stable-sorts all K pairs over 32+ceil(log2 T) bits
// (rasterizer_splat.cu:114-174,473-480): ~6 passes over 12-byte pairs.  The
// resulting order is (tile, depth', gaussian index).  Here the N Gaussians are
// stable-sorted once by depth' (4 passes over N), pairs are emitted in that
// rank order, and a stable sort by tile id alone (ceil(log2 T / 8) passes,
// 2 for T <= 65536) finishes the job: same order, far fewer bytes moved.
#include <cstdlib>
#include <type_traits>

#include "hrf_internal.h"
#include "render_cull.h"

namespace hrf {
namespace {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;  // elements per block

constexpr int kRadixItems = 8;  // keys per thread and tile
// Block size of the radix kernels: 256 threads (2048-key tiles), or 1024
// (8192-key tiles) for sorts of at least kRadixLargeMinKeys keys.  Longer
// tiles give longer output runs per digit, which memory writes more
// efficiently (8.7e8 pairs: 9.6 -> 7.9 ms for the two passes), but fewer,
// longer blocks cost the smaller sorts (1.1e7 pairs: 101 -> 116 us).
constexpr int kRadixThreads = 256;
constexpr int kRadixThreadsLarge = 1024;
constexpr int64_t kRadixLargeMinKeys = int64_t{1} << 26;
constexpr int kRadixTile = kRadixThreads * kRadixItems;  // the smaller tile
constexpr int kRadixBins = 256;
// Partitioning of the radix passes: one tile per block up to
// kRadixTargetParts tiles, beyond that up to kRadixMaxSub tiles per block.
constexpr int kRadixTargetParts = 4096;
// The same for sorts of 2048-key tiles (256-thread blocks): longer
// partitions there (a block walks its next tile's keys in while it ranks
// the current one) measured faster (headline tile sort 94 -> 90 us with
// 1024 against 4096).
constexpr int kRadixTargetPartsSmall = 1024;
constexpr int kRadixMaxSub = 64;

constexpr int kDiffThreads = 1024;
constexpr int kDiffItems = 4;    // Gaussians per thread per step, loads issued together
constexpr int kDiffBlocks = 256;

__device__ __forceinline__ int lane_id() { return __lane_id(); }
// A value that is the same in every lane, moved to scalar registers.
__device__ __forceinline__ int64_t uniform_i64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Exclusive block scan of one value per thread (wave64 shuffles + LDS).
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* total, T* s_wave) {
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  T x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    T y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) s_wave[wave] = x;
  __syncthreads();
  T wave_off = 0, tot = 0;
  const int nw = blockDim.x >> 6;
  for (int w = 0; w < nw; ++w) {
    T t = s_wave[w];
    if (w < wave) wave_off += t;
    tot += t;
  }
  *total = tot;
  return wave_off + x - v;
}

// ----------------------------------------------------------- radix sort --

// The keys are cut into partitions of `sub` consecutive tiles of
// kRadixItems keys per thread of the block (sub grows with n so that the
// partition count stays near kRadixTargetParts): the histogram spine is
// [digit][partition], small enough that its scan is a few coalesced block
// scans, and the scatter block of a partition walks its tiles in order
// carrying each digit's running output offset.

// Digit histogram of each partition: digit = (key >> shift) & mask with at
// most 2^RB values.  The keys come in long runs of equal digits (a
// Gaussian's consecutive tiles), so one histogram per wave made most lanes
// of an atomic add hit one address.  Here the block keeps 16 copies, lane l
// adding into copy l % 16, each copy one padded row (2^RB + 1 words): the
// lanes of a run of equal digits hit 16 different banks, and at most the 4
// lanes l, l+16, l+32, l+48 share an address.  The copies are summed at the
// end.  hist is digit-major ([digit][partition]): a scan along each digit's
// row plus the totals of the lower digits give every (digit, partition)
// output offset.
template <int RB, int TH>
__global__ __launch_bounds__(TH) void k_radix_hist(const uint32_t* __restrict__ keys,
                                                              int64_t n, int shift,
                                                              uint32_t mask,
                                                              uint32_t* __restrict__ hist,
                                                              int nparts, int sub,
                                                              const uint32_t* __restrict__ run_flag) {
  constexpr int kBins = 1 << RB;
  constexpr int kCopies = 16, kRow = kBins + 1, kTile = TH * kRadixItems;
  if (run_flag && *run_flag == 0u) return;
  __shared__ uint32_t s_hist[kCopies * kRow];
  for (int e = threadIdx.x; e < kCopies * kRow; e += TH) s_hist[e] = 0;
  __syncthreads();
  uint32_t* const my_hist = s_hist + (threadIdx.x & (kCopies - 1)) * kRow;
  const int64_t pbase = static_cast<int64_t>(blockIdx.x) * sub * kTile;
  for (int t = 0; t < sub; ++t) {
    const int64_t base = pbase + static_cast<int64_t>(t) * kTile;
    if (base >= n) break;
    uint32_t k[kRadixItems];
#pragma unroll
    for (int i = 0; i < kRadixItems; ++i) {
      const int64_t idx = base + i * TH + threadIdx.x;
      k[i] = idx < n ? keys[idx] : 0u;
    }
#pragma unroll
    for (int i = 0; i < kRadixItems; ++i) {
      const int64_t idx = base + i * TH + threadIdx.x;
      if (idx < n) atomicAdd(&my_hist[(k[i] >> shift) & mask], 1u);
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < kBins; d += TH) {
    uint32_t c = 0;
#pragma unroll
    for (int w = 0; w < kCopies; ++w) c += s_hist[w * kRow + d];
    hist[static_cast<int64_t>(d) * nparts + blockIdx.x] = c;
  }
}

// Per digit (one block each): exclusive scan of the digit's per-partition
// counts across the partitions, in place, and the digit's total.  The row
// is scanned in chunks of kRowScanItems * kRowScanThreads (each thread
// kRowScanItems consecutive counts) with a running carry.  The scatter adds
// the totals of the lower digits itself.
constexpr int kRowScanThreads = 1024;
constexpr int kRowScanItems = 4;
__global__ __launch_bounds__(kRowScanThreads) void k_radix_rowscan(
    uint32_t* __restrict__ hist, int nparts, uint32_t* __restrict__ totals,
    const uint32_t* __restrict__ run_flag) {
  if (run_flag && *run_flag == 0u) return;
  __shared__ uint32_t s_wave[kRowScanThreads / 64];
  uint32_t* row = hist + static_cast<int64_t>(blockIdx.x) * nparts;
  uint32_t carry = 0;
  for (int c0 = 0; c0 < nparts; c0 += kRowScanItems * kRowScanThreads) {
    const int b = c0 + kRowScanItems * static_cast<int>(threadIdx.x);
    uint32_t v[kRowScanItems];
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < kRowScanItems; ++j) {
      v[j] = b + j < nparts ? row[b + j] : 0u;
      sum += v[j];
    }
    uint32_t total;
    uint32_t run = carry + block_exclusive_scan(sum, &total, s_wave);
#pragma unroll
    for (int j = 0; j < kRowScanItems; ++j) {
      if (b + j < nparts) row[b + j] = run;
      run += v[j];
    }
    carry += total;
    __syncthreads();  // s_wave is rewritten by the next chunk's scan
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = carry;
}

// Loads one wave's kRadixItems x 64 consecutive keys (and values) from
// wbase on (wbase and n the same in every lane).  Every lane issues every
// load (indices past n read element n - 1, n > 0): the number of loads in
// flight is then the same on every path, so a wait for them can leave
// later stores outstanding.  The entries past n are never ranked or
// written (rank_tile tests the index).
template <bool VALS>
__device__ __forceinline__ void load_tile(const uint32_t* __restrict__ kin,
                                          const uint32_t* __restrict__ vin, int64_t wbase,
                                          int64_t n, int lane, uint32_t (&key)[kRadixItems],
                                          uint32_t (&val)[kRadixItems]) {
  // Scalar base and last valid offset: past the end the whole wave reads
  // element n - 1.
  const int64_t rem = n - wbase;
  const int64_t b = rem > 0 ? wbase : n - 1;
  const uint32_t lim =
      rem > 0 ? static_cast<uint32_t>(rem < kRadixItems * 64 ? rem : kRadixItems * 64) - 1u : 0u;
  const uint32_t* kw = kin + b;
  if (VALS && vin) {
    const uint32_t* vw = vin + b;
#pragma unroll
    for (int it = 0; it < kRadixItems; ++it) {
      const uint32_t o = static_cast<uint32_t>(it * 64 + lane);
      const uint32_t src = o < lim ? o : lim;
      key[it] = kw[src];
      val[it] = vw[src];
    }
  } else {
    // vin == nullptr: the values are the element indices (first pass of a
    // sort whose payload is the identity permutation).
#pragma unroll
    for (int it = 0; it < kRadixItems; ++it) {
      const uint32_t o = static_cast<uint32_t>(it * 64 + lane);
      key[it] = kw[o < lim ? o : lim];
      if (VALS) val[it] = static_cast<uint32_t>(wbase) + o;
    }
  }
}

// Ranks one wave's loaded keys: rank = the number of keys with the same
// digit before it in the wave's range (the wave's LDS digit counters `cnt`
// carry the count across the items), dig = its digit, or -1 past the end.
// The lanes holding the same digit are found from one ballot per digit bit:
// ANDed over the bits, the ballot where this lane's bit is set, its
// complement where it is clear — b & ~(a ^ c) with a the ballot, b the
// running mask and c all ones or zeros, one three-input bitwise instruction
// per 32-bit half (truth table 0x84, symmetric in a and c).
template <int RB, bool FULL>
__device__ __forceinline__ void rank_tile(const uint32_t (&key)[kRadixItems], int64_t wbase,
                                          int64_t n, int lane, uint64_t lt_mask, int shift,
                                          uint32_t mask, uint32_t* cnt,
                                          uint32_t (&rank)[kRadixItems],
                                          int (&dig)[kRadixItems]) {
#pragma unroll
  for (int it = 0; it < kRadixItems; ++it) {
    const int o = it * 64 + lane;
    const bool valid = FULL || wbase + o < n;
    const uint32_t d = valid ? (key[it] >> shift) & mask : 0u;
    dig[it] = valid ? static_cast<int>(d) : -1;
    const uint64_t vb = FULL ? ~0ull : __ballot(valid);
    uint32_t lo = static_cast<uint32_t>(vb), hi = static_cast<uint32_t>(vb >> 32);
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      // m: all ones where bit b of the digit is set (a sign-extending bit
      // field extract), and the wave's mask of those lanes from one compare
      // (a ballot of an int predicate would be materialised and compared
      // again).
      uint32_t m = static_cast<uint32_t>(static_cast<int32_t>(d << (31 - b)) >> 31);
      asm("" : "+v"(m));  // compare m itself, not the shifted digit again
      const uint64_t bb = __builtin_amdgcn_ballot_w64(m != 0u);
      lo = __builtin_amdgcn_bitop3_b32(static_cast<uint32_t>(bb), lo, m, 0x84);
      hi = __builtin_amdgcn_bitop3_b32(static_cast<uint32_t>(bb >> 32), hi, m, 0x84);
    }
    const uint64_t peers = (static_cast<uint64_t>(hi) << 32) | lo;
    // peers in the lanes below this one (mbcnt: the mask's bits below the
    // lane; lt_mask holds the same lanes)
    const uint32_t before = __builtin_amdgcn_mbcnt_hi(hi, __builtin_amdgcn_mbcnt_lo(lo, 0u));
    uint32_t prev = 0;
    if (valid) prev = cnt[d];
    rank[it] = prev + before;
    if (valid && before == 0) cnt[d] = prev + static_cast<uint32_t>(__popcll(peers));
  }
}

// Digit d's first output position in the pass for partition column `col`
// of the scanned spine (thread d < 2^RB; 0 in the other threads): the
// global totals of the lower digits plus the column's offset along digit
// d's row.  Holds a barrier.
template <int RB>
__device__ __forceinline__ uint32_t digit_run_start(const uint32_t* __restrict__ digit_totals,
                                                    const uint32_t* __restrict__ hist_scan,
                                                    int nparts, int col, int wave, int lane,
                                                    uint32_t* s_wsum) {
  constexpr int kBins = 1 << RB;
  const uint32_t gtot = threadIdx.x < kBins ? digit_totals[threadIdx.x] : 0u;
  uint32_t gincl = gtot;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t gy = __shfl_up(gincl, o, 64);
    if (lane >= o) gincl += gy;
  }
  if (lane == 63) s_wsum[wave] = gincl;
  __syncthreads();
  uint32_t run = 0;
  if (threadIdx.x < kBins) {
    const int d = threadIdx.x;
    uint32_t gbase = gincl - gtot;
    for (int w = 0; w < wave; ++w) gbase += s_wsum[w];
    run = gbase + hist_scan[static_cast<int64_t>(d) * nparts + col];
  }
  return run;
}

// One tile of a stable scatter pass: this lane's kRadixItems keys (and
// values) of the tile at bbase in the wave-contiguous layout (wave w owns
// [bbase + w * 512, + 512), item it at w * 512 + it * 64 + lane), the valid
// ones those below pend (FULL: all kTile).  The keys are ranked by digit
// (ballot match plus per-wave LDS digit counters), reordered by digit in
// LDS (stable: digit, wave, rank) and written from there in order, so
// consecutive threads store consecutive elements of each digit's output
// run.  Thread d < 2^RB holds digit d's next output position (`run`),
// advanced by the digit's count.  The caller has cleared s_cnt before the
// first tile; this clears it again for the next.  narrow >= 0 (with
// values): one word per element into kout, (key >> nshift) << narrow | value
// — the key bits the later passes sort on, above the value's narrow bits.
// tag_out (key writes): word bit 31 of each element as a byte beside it.
template <int RB, bool VALS, int TH, bool FULL>
__device__ __forceinline__ void scatter_tile(
    const uint32_t (&key)[kRadixItems], const uint32_t (&val)[kRadixItems], int64_t bbase,
    int64_t pend, int wave, int lane, uint64_t lt_mask, int shift, uint32_t mask,
    uint32_t (*s_cnt)[1 << RB], uint32_t* s_delta, uint32_t* s_wsum, uint32_t* s_key,
    uint32_t* s_val, uint32_t& run, bool write_keys, uint32_t* __restrict__ kout,
    uint32_t* __restrict__ vout, uint32_t out_mask, int narrow = -1, int nshift = 0,
    uint8_t* __restrict__ tag_out = nullptr) {
  constexpr int kBins = 1 << RB;
  constexpr int kWaves = TH / 64, kTile = TH * kRadixItems;
  const int64_t wbase = bbase + static_cast<int64_t>(wave) * (kRadixItems * 64);
  const int nvalid =
      FULL ? kTile : static_cast<int>(pend - bbase < kTile ? pend - bbase : kTile);
  uint32_t rank[kRadixItems];
  int dig[kRadixItems];
  rank_tile<RB, FULL>(key, wbase, pend, lane, lt_mask, shift, mask, s_cnt[wave], rank, dig);
  __syncthreads();
  // Per digit: the counts of the lower waves (s_cnt becomes each wave's
  // local start), the tile total, and the exclusive scan over the digits
  // of the tile totals (the digit's local start in the reordered tile).
  uint32_t tot = 0;
  if (threadIdx.x < kBins) {
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot += s_cnt[w][threadIdx.x];
  }
  uint32_t incl = tot;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) s_wsum[wave] = incl;
  __syncthreads();
  if (threadIdx.x < kBins) {
    const int d = threadIdx.x;
    uint32_t loc = incl - tot;
    for (int w = 0; w < wave; ++w) loc += s_wsum[w];
    s_delta[d] = run - loc;
    run += tot;
    uint32_t r = loc;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const uint32_t c = s_cnt[w][d];
      s_cnt[w][d] = r;
      r += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < kRadixItems; ++it) {
    if (dig[it] >= 0) {
      const uint32_t lp = s_cnt[wave][dig[it]] + rank[it];
      s_key[lp] = key[it];
      if (VALS) s_val[lp] = val[it];
    }
  }
  __syncthreads();
  // The digit counters are read no more in this tile: clear them for the
  // next one (the barrier after the write-out orders it).
  for (int e = threadIdx.x; e < kWaves * kBins; e += TH)
    s_cnt[e / kBins][e % kBins] = 0;
  if (VALS && narrow >= 0) {
#pragma unroll
    for (int it = 0; it < kRadixItems; ++it) {
      const int i = it * TH + static_cast<int>(threadIdx.x);
      if (FULL || i < nvalid) {
        const uint32_t k = s_key[i];
        const uint32_t pos = s_delta[(k >> shift) & mask] + static_cast<uint32_t>(i);
        kout[pos] = ((k >> nshift) << narrow) | s_val[i];
      }
    }
  } else if (write_keys) {
#pragma unroll
    for (int it = 0; it < kRadixItems; ++it) {
      const int i = it * TH + static_cast<int>(threadIdx.x);
      if (FULL || i < nvalid) {
        const uint32_t k = s_key[i];
        const uint32_t pos = s_delta[(k >> shift) & mask] + static_cast<uint32_t>(i);
        kout[pos] = k & out_mask;
        if (VALS) vout[pos] = s_val[i];
        if (tag_out) tag_out[pos] = static_cast<uint8_t>(k >> 31);
      }
    }
  } else {
#pragma unroll
    for (int it = 0; it < kRadixItems; ++it) {
      const int i = it * TH + static_cast<int>(threadIdx.x);
      if (FULL || i < nvalid) {
        const uint32_t pos = s_delta[(s_key[i] >> shift) & mask] + static_cast<uint32_t>(i);
        vout[pos] = s_val[i];
      }
    }
  }
  // Orders this tile's reads of s_key/s_val/s_delta and the counter
  // clear before the next tile's writes.
  __syncthreads();
}

// Stable scatter of one partition, tile by tile (scatter_tile), each
// tile's keys loaded during the previous tile.  kout == nullptr with VALS:
// only the values are written (the caller needs no sorted keys); narrow >=
// 0: one narrowed word per element into kout (scatter_tile).
template <int RB, bool VALS, int TH>
__global__ __launch_bounds__(TH) void k_radix_scatter(
    const uint32_t* __restrict__ kin, const uint32_t* __restrict__ vin,
    uint32_t* __restrict__ kout, uint32_t* __restrict__ vout, int64_t n, int shift,
    uint32_t mask, const uint32_t* __restrict__ hist_scan,
    const uint32_t* __restrict__ digit_totals, int nparts, int sub,
    const uint32_t* __restrict__ run_flag, uint32_t out_mask,
    const int64_t* __restrict__ bounds, int narrow, int nshift, uint8_t* __restrict__ tag_out) {
  constexpr int kBins = 1 << RB;
  constexpr int kWaves = TH / 64, kTile = TH * kRadixItems;
  static_assert(kBins <= TH, "one thread per digit");
  if (run_flag && *run_flag == 0u) return;
  __shared__ uint32_t s_cnt[kWaves][kBins];
  __shared__ uint32_t s_delta[kBins];  // output offset of the digit minus its local offset
  __shared__ uint32_t s_wsum[kWaves];
  __shared__ uint32_t s_key[kTile];
  __shared__ uint32_t s_val[VALS ? kTile : 1];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const bool write_keys = !VALS || kout != nullptr;

  // The partition's first spine column is its first emission block when
  // `bounds` gives the partitions.
  const int col = bounds ? static_cast<int>(blockIdx.x) * sub : static_cast<int>(blockIdx.x);
  uint32_t run = digit_run_start<RB>(digit_totals, hist_scan, nparts, col, wave, lane, s_wsum);
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));

  // This block's partition [pstart, pend): sub tiles from blockIdx.x * sub,
  // or (bounds) the pairs of emission blocks [blockIdx.x * sub, + sub).
  int64_t pstart, pend;
  if (bounds) {
    const int b0 = static_cast<int>(blockIdx.x) * sub;
    const int b1 = b0 + sub < nparts ? b0 + sub : nparts;
    pstart = bounds[b0] < n ? bounds[b0] : n;
    pend = bounds[b1] < n ? bounds[b1] : n;
  } else {
    pstart = static_cast<int64_t>(blockIdx.x) * sub * kTile;
    pend = pstart + static_cast<int64_t>(sub) * kTile < n
               ? pstart + static_cast<int64_t>(sub) * kTile
               : n;
  }
  // The same in every lane: held as scalars, so the tile loop and its
  // full/partial choice are scalar branches.
  pstart = uniform_i64(pstart);
  pend = uniform_i64(pend);

  for (int e = threadIdx.x; e < kWaves * kBins; e += TH)
    s_cnt[e / kBins][e % kBins] = 0;
  __syncthreads();
  // The keys (and values) of the next tile are loaded while this one is
  // ranked and written: each tile's load latency hides behind the previous
  // tile's work instead of adding to it.
  const int64_t woff = static_cast<int64_t>(wave) * (kRadixItems * 64);
  uint32_t key[kRadixItems], val[kRadixItems], nkey[kRadixItems], nval[kRadixItems];
  int64_t bbase = pstart;
  if (bbase < pend) load_tile<VALS>(kin, vin, bbase + woff, pend, lane, nkey, nval);
  for (; bbase + kTile <= pend; bbase += kTile) {
#pragma unroll
    for (int it = 0; it < kRadixItems; ++it) {
      key[it] = nkey[it];
      val[it] = nval[it];
    }
    if (bbase + kTile < pend)
      load_tile<VALS>(kin, vin, bbase + kTile + woff, pend, lane, nkey, nval);
    scatter_tile<RB, VALS, TH, true>(key, val, bbase, pend, wave, lane, lt_mask, shift, mask,
                                     s_cnt, s_delta, s_wsum, s_key, s_val, run, write_keys,
                                     kout, vout, out_mask, narrow, nshift, tag_out);
  }
  if (bbase < pend)
    scatter_tile<RB, VALS, TH, false>(nkey, nval, bbase, pend, wave, lane, lt_mask, shift, mask,
                                      s_cnt, s_delta, s_wsum, s_key, s_val, run, write_keys,
                                      kout, vout, out_mask, narrow, nshift, tag_out);
}

__global__ void k_fill_u32(uint32_t* p, uint32_t v, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void k_fill_f32(float* p, float v, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// 16-byte-aligned fill: kFillVec float4 stores per thread, grid-strided.
constexpr int kFillVec = 4;
__global__ __launch_bounds__(256) void k_fill_f32x4(float4* p, float v, int64_t n4) {
  const float4 q = make_float4(v, v, v, v);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
#pragma unroll
  for (int k = 0; k < kFillVec; ++k, i += stride)
    if (i < n4) p[i] = q;
}

// Depth-order permutation: order[i] when the depth sort ran (*sorted_flag
// != 0), the identity otherwise (the keys were already in order).
__device__ __forceinline__ uint32_t ordered(const uint32_t* order, const uint32_t* sorted_flag,
                                           int64_t i) {
  return *sorted_flag ? order[i] : static_cast<uint32_t>(i);
}

// Pair and visible offsets (three launches for both scans).  Pair counts
// are taken in depth-rank order (tiles[order[i]], or tiles[i] with no
// order), visibility flags in index order.
//   k_offsets_reduce: per-block sums of both arrays;
//   k_offsets_blocks: one block scans the block sums in place (exclusive) and
//     writes the totals [K, V, *sort_flag] and off[n] = K;
//   k_offsets_scan: per-block exclusive scans plus the block prefixes.
__device__ __forceinline__ void load_counts(const uint32_t* __restrict__ order,
                                            const uint32_t* __restrict__ tiles,
                                            const uint32_t* __restrict__ vis, int64_t n,
                                            int64_t base, uint32_t (&t)[kScanItems],
                                            uint32_t (&v)[kScanItems]) {
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    const int64_t idx = base + i;
    t[i] = 0u;
    v[i] = 0u;
    if (idx < n) {
      t[i] = tiles[order ? order[idx] : static_cast<uint32_t>(idx)];
      v[i] = vis[idx];
    }
  }
}

__global__ __launch_bounds__(kScanThreads) void k_offsets_reduce(
    const uint32_t* __restrict__ order, const uint32_t* __restrict__ tiles,
    const uint32_t* __restrict__ vis, int64_t n, uint64_t* __restrict__ bsum_p,
    uint32_t* __restrict__ bsum_v) {
  __shared__ uint64_t s_p[kScanThreads / 64];
  __shared__ uint32_t s_v[kScanThreads / 64];
  uint32_t t[kScanItems], v[kScanItems];
  load_counts(order, tiles, vis, n,
              static_cast<int64_t>(blockIdx.x) * kScanTile +
                  static_cast<int64_t>(threadIdx.x) * kScanItems,
              t, v);
  uint64_t sp = 0;
  uint32_t sv = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    sp += t[i];
    sv += v[i];
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    sp += __shfl_xor(sp, d, 64);
    sv += __shfl_xor(sv, d, 64);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_p[wave] = sp;
    s_v[wave] = sv;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t a = 0;
    uint32_t b = 0;
#pragma unroll
    for (int w = 0; w < kScanThreads / 64; ++w) {
      a += s_p[w];
      b += s_v[w];
    }
    bsum_p[blockIdx.x] = a;
    bsum_v[blockIdx.x] = b;
  }
}

template <int THREADS = kScanThreads, int ITEMS = kScanItems>
__global__ __launch_bounds__(THREADS) void k_offsets_blocks(
    uint64_t* __restrict__ bsum_p, uint32_t* __restrict__ bsum_v, int64_t nb,
    uint64_t* __restrict__ off_end, const uint32_t* __restrict__ sort_flag,
    uint64_t* __restrict__ totals, uint32_t* __restrict__ flag_out, uint64_t tag) {
  __shared__ uint64_t s_wp[THREADS / 64];
  __shared__ uint32_t s_wv[THREADS / 64];
  uint64_t carry_p = 0;
  uint32_t carry_v = 0;
  uint32_t flags = 0;  // with flag_out: OR of the kPartFlag bits of bsum_v
  for (int64_t base = 0; base < nb; base += THREADS * ITEMS) {
    const int64_t b0 = base + static_cast<int64_t>(threadIdx.x) * ITEMS;
    uint64_t p[ITEMS];
    uint32_t v[ITEMS];
    uint64_t rp = 0;
    uint32_t rv = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int64_t idx = b0 + i;
      const uint64_t xp = idx < nb ? bsum_p[idx] : 0ull;
      uint32_t xv = (bsum_v && idx < nb) ? bsum_v[idx] : 0u;
      if (flag_out) {
        flags |= xv;
        xv &= ~kPartFlag;
      }
      p[i] = rp;
      v[i] = rv;
      rp += xp;
      rv += xv;
    }
    uint64_t tp;
    uint32_t tv;
    const uint64_t op = block_exclusive_scan<uint64_t>(rp, &tp, s_wp);
    const uint32_t ov = block_exclusive_scan<uint32_t>(rv, &tv, s_wv);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int64_t idx = b0 + i;
      if (idx < nb) {
        bsum_p[idx] = carry_p + op + p[i];
        if (bsum_v) bsum_v[idx] = carry_v + ov + v[i];
      }
    }
    carry_p += tp;
    carry_v += tv;
    __syncthreads();  // s_wp / s_wv are reused by the next chunk
  }
  uint32_t flag = 0;
  if (flag_out) flag = __syncthreads_or((flags & kPartFlag) != 0 ? 1 : 0) != 0 ? 1u : 0u;
  if (threadIdx.x == 0) {
    off_end[0] = carry_p;
    if (flag_out) *flag_out = flag;
    if (totals) {
      totals[0] = carry_p;
      totals[1] = carry_v;
      totals[2] = flag_out ? flag : *sort_flag;
      if (tag) {
        // the counts reach the host (system scope) before the tag does
        __threadfence_system();
        totals[3] = tag;
      }
    }
  }
}

// Tile counts per kProjThreads block of ranks, taken in rank order.
__global__ __launch_bounds__(kProjThreads) void k_rank_partials(const uint32_t* __restrict__ order,
                                                               const uint32_t* __restrict__ tiles,
                                                               int64_t n,
                                                               uint64_t* __restrict__ part_r) {
  __shared__ uint64_t s_t[kProjThreads / 64];
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kProjThreads + threadIdx.x;
  uint64_t t = r < n ? tiles[order[r]] : 0u;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) t += __shfl_xor(t, d, 64);
  if ((threadIdx.x & 63) == 0) s_t[threadIdx.x >> 6] = t;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t a = 0;
#pragma unroll
    for (int w = 0; w < kProjThreads / 64; ++w) a += s_t[w];
    part_r[blockIdx.x] = a;
  }
}

// The block's exclusive pair offsets (kProjThreads ranks) from its tile
// counts and the scanned base: s_off[0..nr], s_off[nr] = the next block's
// base.  Every thread of the block calls it (it synchronises).
__device__ __forceinline__ void block_offsets(const uint64_t* __restrict__ part_t,
                                              const uint64_t* __restrict__ part_r,
                                              const uint32_t* __restrict__ tiles,
                                              const uint32_t* __restrict__ order,
                                              const uint32_t* __restrict__ sorted_flag,
                                              int64_t rb, int nr, uint64_t* s_off,
                                              uint64_t* s_wave) {
  const bool ranked = *sorted_flag != 0;
  const uint64_t* base = ranked ? part_r : part_t;
  const int64_t r = rb + threadIdx.x;
  uint64_t c = 0;
  if (static_cast<int>(threadIdx.x) < nr)
    c = tiles[ranked ? order[r] : static_cast<uint32_t>(r)];
  uint64_t total;
  const uint64_t ex = block_exclusive_scan<uint64_t>(c, &total, s_wave);
  const uint64_t b0 = base[blockIdx.x];
  if (static_cast<int>(threadIdx.x) < nr) s_off[threadIdx.x] = b0 + ex;
  if (threadIdx.x == 0) s_off[nr] = b0 + total;
}

__global__ __launch_bounds__(kScanThreads) void k_offsets_scan(
    const uint32_t* __restrict__ order, const uint32_t* __restrict__ tiles,
    const uint32_t* __restrict__ vis, int64_t n, const uint64_t* __restrict__ bsum_p,
    const uint32_t* __restrict__ bsum_v, uint64_t* __restrict__ off,
    uint32_t* __restrict__ vis_off) {
  __shared__ uint64_t s_wp[kScanThreads / 64];
  __shared__ uint32_t s_wv[kScanThreads / 64];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile +
                       static_cast<int64_t>(threadIdx.x) * kScanItems;
  uint32_t t[kScanItems], v[kScanItems];
  load_counts(order, tiles, vis, n, base, t, v);
  uint64_t p[kScanItems];
  uint32_t q[kScanItems];
  uint64_t rp = 0;
  uint32_t rv = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    p[i] = rp;
    q[i] = rv;
    rp += t[i];
    rv += v[i];
  }
  uint64_t tp;
  uint32_t tv;
  const uint64_t op = block_exclusive_scan<uint64_t>(rp, &tp, s_wp) + bsum_p[blockIdx.x];
  const uint32_t ov = block_exclusive_scan<uint32_t>(rv, &tv, s_wv) + bsum_v[blockIdx.x];
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    const int64_t idx = base + i;
    if (idx < n) {
      off[idx] = op + p[i];
      vis_off[idx] = ov + q[i];
    }
  }
}

// Pairs [a, a + cnt) of an emission block, whose pair offsets are
// s_off[0..nr] and whose Gaussians and packed rectangles are s_g and s_rect
// (rank order), handed to store(j, tile id, gaussian, the gaussian's index
// in the block, tile x, tile y) for j = 0..cnt-1: one
// binary search finds the first pair's Gaussian and tile (one division by
// the rectangle width), then a walk goes on (next tile of the rectangle, y
// outer and x inner as rasterizer_splat.cu:162-173 emits them; next
// Gaussian with pairs).
template <typename Store>
__device__ __forceinline__ void walk_pairs(uint64_t a, int cnt, const uint64_t* s_off, int nr,
                                           const uint2* s_rect, const uint32_t* s_g, uint32_t ugx,
                                           Store store) {
  int lo = 0, hi = nr;  // the largest lo with s_off[lo] <= a: a < s_off[lo + 1]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (s_off[mid] <= a)
      lo = mid;
    else
      hi = mid;
  }
  uint64_t next = s_off[lo + 1];
  uint2 rc = s_rect[lo];
  uint32_t minx = rc.x & 0xFFFF, maxx = rc.y & 0xFFFF;
  const uint32_t w0 = maxx - minx;
  const uint32_t i0 = static_cast<uint32_t>(a - s_off[lo]);
  uint32_t ty = (rc.x >> 16) + i0 / w0, tx = minx + i0 % w0;
  uint32_t gb = s_g[lo];
  for (int j = 0; j < cnt; ++j) {
    const uint64_t e = a + j;
    if (e == next) {  // this Gaussian is done: the next one with pairs
      do {
        ++lo;
        next = s_off[lo + 1];
      } while (next == e);
      rc = s_rect[lo];
      minx = rc.x & 0xFFFF;
      maxx = rc.y & 0xFFFF;
      tx = minx;
      ty = rc.x >> 16;
      gb = s_g[lo];
    }
    store(j, ty * ugx + tx, gb, lo, tx, ty);
    if (++tx == maxx) {
      tx = minx;
      ++ty;
    }
  }
}

// Pair emission.  A block owns kEmitThreads consecutive ranks; it forms
// their exclusive pair offsets in LDS (a block scan of their tile counts
// plus the block's scanned base) and writes the block's output range
// [off[r_begin], off[r_end]).  Tile order inside a Gaussian is y outer, x
// inner (rasterizer_splat.cu:162-173).
constexpr int kEmitThreads = kProjThreads;
// Visible compaction of index block blockIdx.x (indices [256 b, 256 b +
// 256), the block base part_v[b] from the scan), done by the emission
// launch, whose grid has the same blocks: every thread of the block calls
// it.
struct VisibleOut {
  const uint32_t* vis;
  const uint32_t* part_v;
  int64_t* visible;  // nullptr: nothing to write
  int64_t vmax;      // length of `visible`: positions at or past it are not written
};

__device__ __forceinline__ void compact_visible_block(const VisibleOut& vo, int64_t n) {
  if (!vo.visible) return;
  __shared__ uint32_t s_vw[kEmitThreads / 64];
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kEmitThreads + threadIdx.x;
  const uint32_t v = i < n ? vo.vis[i] : 0u;
  uint32_t total;
  const uint32_t ex = block_exclusive_scan<uint32_t>(v, &total, s_vw);
  const int64_t at = static_cast<int64_t>(vo.part_v[blockIdx.x]) + ex;
  if (v && at < vo.vmax) vo.visible[at] = i;
}

// The block's pairs [e0, e1) (those of its kEmitThreads Gaussians in rank
// order) are produced in chunks of kEmitChunk: each thread takes kEmitPer
// consecutive pairs, finds the Gaussian and tile of its first one (one
// binary search over the block's offsets, one division by the rect width),
// then walks on (next tile in the rect, next Gaussian with pairs) and stores
// the pairs in LDS (one pad word per kEmitPer, so the lanes' strided stores
// hit distinct banks); the chunk then leaves in coalesced stores.
// kWide == false: one word (tile << vbits) | gaussian per pair into
// `words`.  kWide: the tile id into `words` and the gaussian into `vals`
// (tile and gaussian bits do not fit one word).  kStore == false (with
// kHist): the pairs are only counted for the first sort pass's histogram;
// k_emit_scatter regenerates and scatters them.
// (8 pairs per thread: 18.5 KB of LDS per block, 8 blocks per CU; 16
// measured slower for config 2, 26 against 21.5 us, with 26.7 KB and 6.)
constexpr int kEmitPer = 8;
constexpr int kEmitChunk = kEmitThreads * kEmitPer;
__device__ __forceinline__ int emit_pad(int i) { return i + i / kEmitPer; }

// Optional first sort pass histogram taken by the emission: each emission
// block is then one partition of that pass (its pairs [e0, e1)).  hist
// (digit-major, gridDim.x columns) receives the block's counts of digit
// (key >> shift) & mask; bounds[b] the block's first pair, bounds[gridDim.x]
// the pair count.
struct EmitHist {
  uint32_t* hist;  // nullptr: no histogram
  int64_t* bounds;
  int shift;
  uint32_t mask;
  int rows;  // digit rows of the pass's histogram (2^RB >= mask + 1; the rest are zero)
};

template <bool kWide, bool kHist, bool kStore = true>
__global__ __launch_bounds__(kEmitThreads) void k_emit_packed(
    const uint64_t* __restrict__ part_t, const uint64_t* __restrict__ part_r,
    const uint32_t* __restrict__ tiles, const uint32_t* __restrict__ order,
    const uint32_t* __restrict__ sorted_flag, const uint2* __restrict__ rect, int64_t n,
    int64_t k, int gx, int vbits, uint32_t* __restrict__ words, uint32_t* __restrict__ vals,
    VisibleOut vo, EmitHist eh) {
  compact_visible_block(vo, n);
  // (one more slot per wave: the counting path's difference arrays)
  __shared__ uint32_t s_dh[kHist ? kEmitThreads / 64 : 1][kHist ? kRadixBins + 1 : 1];
  const int wave = threadIdx.x >> 6;
  if (kHist) {
    for (int e = threadIdx.x; e < (kEmitThreads / 64) * (kRadixBins + 1); e += kEmitThreads)
      s_dh[e / (kRadixBins + 1)][e % (kRadixBins + 1)] = 0u;
  }
  __shared__ uint64_t s_off[kEmitThreads + 1];
  __shared__ uint32_t s_g[kEmitThreads];
  __shared__ uint2 s_rect[kEmitThreads];
  __shared__ uint32_t s_words[kEmitChunk + kEmitChunk / kEmitPer];
  __shared__ uint32_t s_vals[kWide ? kEmitChunk + kEmitChunk / kEmitPer : 1];
  __shared__ uint64_t s_wave[kEmitThreads / 64];
  const int64_t rb = static_cast<int64_t>(blockIdx.x) * kEmitThreads;
  const int64_t r = rb + threadIdx.x;
  const int nr = static_cast<int>(n - rb < kEmitThreads ? n - rb : kEmitThreads);
  block_offsets(part_t, part_r, tiles, order, sorted_flag, rb, nr, s_off, s_wave);
  if (threadIdx.x < nr) {
    const uint32_t g = ordered(order, sorted_flag, r);
    s_g[threadIdx.x] = g;
    s_rect[threadIdx.x] = rect[g];
  }
  __syncthreads();
  // Pairs at or past k (the output length) are not written.
  const uint64_t uk = static_cast<uint64_t>(k);
  const uint64_t e0 = s_off[0], e1 = s_off[nr] < uk ? s_off[nr] : uk;
  const uint32_t ugx = static_cast<uint32_t>(gx);
  if (!kStore && s_off[nr] <= uk) {
    // Counting only, every pair of the block below k: a Gaussian's pairs
    // are the rows of its tile rectangle, each row a run of consecutive
    // tile ids, and the first digit is the tile id's low bits (eh.shift
    // selects them in both key layouts), so a row adds whole cycles of the
    // 2^bits digits plus one cyclic digit range: a difference array per
    // wave (two to four LDS atomics per row, none per pair), then a scan
    // over the digits.
    __shared__ uint32_t s_wv1[kEmitThreads / 64], s_wv2[kEmitThreads / 64];
    const uint32_t M = eh.mask + 1u;
    uint32_t full = 0;
    if (static_cast<int>(threadIdx.x) < nr && s_off[threadIdx.x + 1] > s_off[threadIdx.x]) {
      const uint2 rc = s_rect[threadIdx.x];
      const uint32_t minx = rc.x & 0xFFFF, maxx = rc.y & 0xFFFF;
      const uint32_t miny = rc.x >> 16, maxy = rc.y >> 16;
      const uint32_t L = maxx - minx, rem = L & eh.mask;
      full = (L / M) * (maxy - miny);
      if (rem) {
        for (uint32_t ty = miny; ty < maxy; ++ty) {
          const uint32_t a = (ty * ugx + minx) & eh.mask, b = a + rem;
          atomicAdd(&s_dh[wave][a], 1u);
          if (b <= M) {
            atomicAdd(&s_dh[wave][b], 0xFFFFFFFFu);
          } else {
            atomicAdd(&s_dh[wave][M], 0xFFFFFFFFu);
            atomicAdd(&s_dh[wave][0], 1u);
            atomicAdd(&s_dh[wave][b - M], 0xFFFFFFFFu);
          }
        }
      }
    }
    uint32_t ftot;
    block_exclusive_scan<uint32_t>(full, &ftot, s_wv1);  // the block's whole cycles
    __syncthreads();
    const int d = static_cast<int>(threadIdx.x);
    uint32_t v = 0;
    if (d <= static_cast<int>(eh.mask)) {
#pragma unroll
      for (int w = 0; w < kEmitThreads / 64; ++w) v += s_dh[w][d];
    }
    uint32_t vtot;
    const uint32_t incl = block_exclusive_scan<uint32_t>(v, &vtot, s_wv2) + v;
    for (int r = d; r < eh.rows; r += kEmitThreads)
      eh.hist[static_cast<int64_t>(r) * gridDim.x + blockIdx.x] =
          r <= static_cast<int>(eh.mask) ? incl + ftot : 0u;
    if (threadIdx.x == 0) {
      eh.bounds[blockIdx.x] = static_cast<int64_t>(e0);
      if (blockIdx.x == gridDim.x - 1) eh.bounds[gridDim.x] = k;
    }
    return;
  }
  for (uint64_t c0 = e0; c0 < e1; c0 += kEmitChunk) {
    const int clen = static_cast<int>(e1 - c0 < kEmitChunk ? e1 - c0 : kEmitChunk);
    const int j0 = static_cast<int>(threadIdx.x) * kEmitPer;
    if (j0 < clen) {
      const int cnt = clen - j0 < kEmitPer ? clen - j0 : kEmitPer;
      walk_pairs(c0 + j0, cnt, s_off, nr, s_rect, s_g, ugx,
                 [&](int j, uint32_t tile, uint32_t gb, int, uint32_t, uint32_t) {
        if (kWide) {
          s_words[emit_pad(j0 + j)] = tile;
          s_vals[emit_pad(j0 + j)] = gb;
        } else {
          s_words[emit_pad(j0 + j)] = (tile << vbits) | gb;
        }
      });
    }
    __syncthreads();
    for (int i = threadIdx.x; i < clen; i += kEmitThreads) {
      const uint32_t w = s_words[emit_pad(i)];
      if (kStore) {
        words[c0 + i] = w;
        if (kWide) vals[c0 + i] = s_vals[emit_pad(i)];
      }
      if (kHist) atomicAdd(&s_dh[wave][(w >> eh.shift) & eh.mask], 1u);
    }
    __syncthreads();
  }
  if (kHist) {
    for (int d = threadIdx.x; d < eh.rows; d += kEmitThreads) {
      uint32_t c = 0;
      if (d <= static_cast<int>(eh.mask)) {
#pragma unroll
        for (int w = 0; w < kEmitThreads / 64; ++w) c += s_dh[w][d];
      }
      eh.hist[static_cast<int64_t>(d) * gridDim.x + blockIdx.x] = c;
    }
    if (threadIdx.x == 0) {
      eh.bounds[blockIdx.x] = static_cast<int64_t>(e0);
      if (blockIdx.x == gridDim.x - 1) eh.bounds[gridDim.x] = k;
    }
  }
}

// The pair emission fused with the first tile-sort pass (large sorts): the
// counting launch (k_emit_packed<kWide, true, false>) has taken the pass's
// digit histogram and partition bounds over the emission blocks and stored
// no pair.  Block b regenerates emission block b's pairs tile by tile (each
// thread walks kRadixItems consecutive pairs of the tile into LDS) and
// scatters each tile by the first digit as k_radix_scatter does a loaded
// one: one write of the pairs instead of a write, a read and a write.
// The partition is [s_off[0], min(s_off[nr], k)), as the counting launch
// recorded it; its spine column is b.  The generated tile is stored at
// index i ^ ((i >> 6) & 7): a thread's 8 consecutive pairs then hit
// distinct banks across the wave (lane t writes 8t + (j ^ (t >> 3))), and
// the scatter's reads (64 consecutive items per wave) stay one contiguous
// run, so the tile needs no padding.
// Wide keys with ts.rec set: each pair's value carries in bit 31 whether
// the forward keeps the gaussian in that tile in some plane (pair_visible;
// the gaussians' cull keys staged in LDS), and the last sort pass writes
// that bit beside point_list for the forward.
template <bool kWide, int RB, int TH>
__global__ __launch_bounds__(TH) void k_emit_scatter(
    const uint64_t* __restrict__ part_t, const uint64_t* __restrict__ part_r,
    const uint32_t* __restrict__ tiles, const uint32_t* __restrict__ order,
    const uint32_t* __restrict__ sorted_flag, const uint2* __restrict__ rect, int64_t n,
    int64_t k, int gx, int vbits, uint32_t* __restrict__ kout, uint32_t* __restrict__ vout,
    int shift, uint32_t mask, const uint32_t* __restrict__ hist_scan,
    const uint32_t* __restrict__ digit_totals, int nparts, int narrow, int nshift, TagSrc ts) {
  constexpr bool VALS = kWide;
  constexpr int kBins = 1 << RB;
  constexpr int kWaves = TH / 64, kTile = TH * kRadixItems;
  static_assert(kBins <= TH && kEmitThreads <= TH, "one thread per digit and per rank");
  static_assert(kRadixItems == 8, "the swizzle assumes 8 items per thread");
  __shared__ uint32_t s_cnt[kWaves][kBins];
  __shared__ uint32_t s_delta[kBins];
  __shared__ uint32_t s_wsum[kWaves];
  __shared__ uint32_t s_key[kTile];
  __shared__ uint32_t s_val[VALS ? kTile : 1];
  __shared__ uint64_t s_off[kEmitThreads + 1];
  __shared__ uint32_t s_g[kEmitThreads];
  __shared__ uint2 s_rect[kEmitThreads];
  __shared__ uint64_t s_wave[kWaves];
  __shared__ CullKey s_ck[kWide ? kEmitThreads : 1];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  uint32_t run = digit_run_start<RB>(digit_totals, hist_scan, nparts,
                                     static_cast<int>(blockIdx.x), wave, lane, s_wsum);
  const bool tagged = kWide && ts.rec != nullptr;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));

  const int64_t rb = static_cast<int64_t>(blockIdx.x) * kEmitThreads;
  const int nr = static_cast<int>(n - rb < kEmitThreads ? n - rb : kEmitThreads);
  block_offsets(part_t, part_r, tiles, order, sorted_flag, rb, nr, s_off, s_wave);
  if (static_cast<int>(threadIdx.x) < nr) {
    const uint32_t g = ordered(order, sorted_flag, rb + threadIdx.x);
    s_g[threadIdx.x] = g;
    s_rect[threadIdx.x] = rect[g];
    if (tagged) {
      const float4* r4 = reinterpret_cast<const float4*>(
          ts.rec + static_cast<int64_t>(g) * ts.rec_stride);
      s_ck[kWide ? threadIdx.x : 0] =
          cull_key(r4[0], r4[1], ts.pprobs + static_cast<int64_t>(g) * ts.P, ts.P);
    }
  }
  for (int e = threadIdx.x; e < kWaves * kBins; e += TH) s_cnt[e / kBins][e % kBins] = 0;
  __syncthreads();
  const int64_t e0 = uniform_i64(static_cast<int64_t>(s_off[0]));
  const int64_t e1 = uniform_i64(static_cast<int64_t>(
      s_off[nr] < static_cast<uint64_t>(k) ? s_off[nr] : static_cast<uint64_t>(k)));
  const uint32_t ugx = static_cast<uint32_t>(gx);
  const int j0 = static_cast<int>(threadIdx.x) * kRadixItems;
  for (int64_t c0 = e0; c0 < e1; c0 += kTile) {
    const int clen = static_cast<int>(e1 - c0 < kTile ? e1 - c0 : kTile);
    if (j0 < clen) {
      const int cnt = clen - j0 < kRadixItems ? clen - j0 : kRadixItems;
      // The cull key of the gaussian being walked, reloaded only when the
      // walk moves on to the next one.
      int ck_lo = -1;
      CullKey ck{};
      walk_pairs(static_cast<uint64_t>(c0 + j0), cnt, s_off, nr, s_rect, s_g, ugx,
                 [&](int j, uint32_t tile, uint32_t gb, int lo, uint32_t tx, uint32_t ty) {
                   const int i = j0 + j;
                   const int sw = i ^ ((i >> 6) & 7);
                   s_key[sw] = kWide ? tile : ((tile << vbits) | gb);
                   if (VALS) {
                     uint32_t v = gb;
                     if (tagged) {
                       if (lo != ck_lo) {
                         ck = s_ck[kWide ? lo : 0];
                         ck_lo = lo;
                       }
                       if (pair_visible(ck, static_cast<float>(tx * hrf::kTile),
                                        static_cast<float>(ty * hrf::kTile)))
                         v |= 0x80000000u;
                     }
                     s_val[sw] = v;
                   }
                 });
    }
    __syncthreads();
    // This lane's items in the scatter's wave-contiguous layout (entries
    // past clen are read but never ranked or written).
    uint32_t key[kRadixItems], val[kRadixItems];
#pragma unroll
    for (int it = 0; it < kRadixItems; ++it) {
      const int i = wave * (kRadixItems * 64) + it * 64 + lane;
      const int sw = i ^ ((i >> 6) & 7);
      key[it] = s_key[sw];
      val[it] = VALS ? s_val[sw] : 0u;
    }
    // scatter_tile's first barrier orders these reads before its reorder
    // writes; its last one orders its reads before the next generation.
    if (clen == kTile)
      scatter_tile<RB, VALS, TH, true>(key, val, c0, e1, wave, lane, lt_mask, shift, mask, s_cnt,
                                       s_delta, s_wsum, s_key, s_val, run, true, kout, vout,
                                       0xFFFFFFFFu, narrow, nshift);
    else
      scatter_tile<RB, VALS, TH, false>(key, val, c0, e1, wave, lane, lt_mask, shift, mask, s_cnt,
                                        s_delta, s_wsum, s_key, s_val, run, true, kout, vout,
                                        0xFFFFFFFFu, narrow, nshift);
  }
}

// Sorted packed words -> point_list (the gaussian field) and tile ranges.
__global__ void k_unpack_ranges(const uint32_t* __restrict__ words, int64_t k, int vbits,
                                int32_t* __restrict__ point_list, int32_t* __restrict__ ranges,
                                uint32_t ntiles) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= k) return;
  const uint32_t w = words[i];
  const uint32_t t = w >> vbits;
  point_list[i] = static_cast<int32_t>(w & ((1u << vbits) - 1u));
  if (t >= ntiles) return;  // only a word the emission never wrote
  if (i == 0 || (words[i - 1] >> vbits) != t)
    ranges[2 * static_cast<int64_t>(t)] = static_cast<int32_t>(i);
  if (i == k - 1 || (words[i + 1] >> vbits) != t)
    ranges[2 * static_cast<int64_t>(t) + 1] = static_cast<int32_t>(i + 1);
}

__global__ void k_tile_ranges(const uint32_t* __restrict__ keys, int64_t k,
                              int32_t* __restrict__ ranges, uint32_t ntiles) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= k) return;
  const uint32_t t = keys[i];
  if (t >= ntiles) return;  // only a key the emission never wrote
  if (i == 0 || keys[i - 1] != t) ranges[2 * static_cast<int64_t>(t)] = static_cast<int32_t>(i);
  if (i == k - 1 || keys[i + 1] != t)
    ranges[2 * static_cast<int64_t>(t) + 1] = static_cast<int32_t>(i + 1);
}

// Tile ranges without reading the sorted pairs.  Gaussian g emits one pair
// per tile of its rectangle [minx, maxx) x [miny, maxy), so the pair count
// of a tile is the number of rectangles covering it: a 2-D difference array
// (+1 at (miny, minx) and (maxy, maxx), -1 at (miny, maxx) and (maxy, minx))
// integrated twice.  Sorted by tile id, tile t's pairs start at the sum of
// the counts of tiles < t.  Blocks accumulate the difference array in LDS
// and flush it with one global atomic per nonzero entry.
__global__ __launch_bounds__(kDiffThreads) void k_tile_diff(const uint32_t* __restrict__ tiles,
                                                           const uint2* __restrict__ rect,
                                                           int64_t n, int gx, int dn,
                                                           int32_t* __restrict__ diff) {
  extern __shared__ int32_t s_diff[];
  for (int e = threadIdx.x; e < dn; e += kDiffThreads) s_diff[e] = 0;
  __syncthreads();
  const int gw = gx + 1;
  constexpr int kPer = kDiffItems * kDiffThreads;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kPer; base < n;
       base += static_cast<int64_t>(gridDim.x) * kPer) {
    uint32_t t[kDiffItems];
    uint2 r[kDiffItems];
#pragma unroll
    for (int j = 0; j < kDiffItems; ++j) {
      const int64_t g = base + j * kDiffThreads + threadIdx.x;
      t[j] = g < n ? tiles[g] : 0u;
      r[j] = g < n ? rect[g] : make_uint2(0u, 0u);
    }
#pragma unroll
    for (int j = 0; j < kDiffItems; ++j) {
      if (t[j] == 0u) continue;
      const int x0 = static_cast<int>(r[j].x & 0xFFFF), y0 = static_cast<int>(r[j].x >> 16);
      const int x1 = static_cast<int>(r[j].y & 0xFFFF), y1 = static_cast<int>(r[j].y >> 16);
      atomicAdd(&s_diff[y0 * gw + x0], 1);
      atomicAdd(&s_diff[y0 * gw + x1], -1);
      atomicAdd(&s_diff[y1 * gw + x0], -1);
      atomicAdd(&s_diff[y1 * gw + x1], 1);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < dn; e += kDiffThreads) {
    const int32_t v = s_diff[e];
    if (v != 0) atomicAdd(&diff[e], v);
  }
}

// Inclusive prefix sum of `len` LDS entries at stride `step` by one wave,
// in chunks of 64 with a carry.
__device__ __forceinline__ void wave_prefix_lds(int32_t* p, int len, int step) {
  const int lane = threadIdx.x & 63;
  int32_t carry = 0;
  for (int c0 = 0; c0 < len; c0 += 64) {
    const int i = c0 + lane;
    int32_t v = i < len ? p[i * step] : 0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int32_t y = __shfl_up(v, o, 64);
      if (lane >= o) v += y;
    }
    v += carry;
    if (i < len) p[i * step] = v;
    carry = __shfl(v, 63, 64);
  }
}

// One block: integrate the difference array (rows, then columns, one wave
// per line), then an exclusive scan of the counts in tile order; empty
// tiles get (0, 0), as a zero-filled ranges buffer has for tiles without
// pairs.
// With tile_order: also the tile ids by list length, longest first (256
// logarithmic buckets, cost_bucket; arbitrary order within a bucket), for
// the forward render's block order.
__global__ __launch_bounds__(kDiffThreads) void k_ranges_from_diff(const int32_t* __restrict__ diff,
                                                                  int gx, int gy,
                                                                  int32_t* __restrict__ ranges,
                                                                  int32_t* __restrict__ tile_order) {
  extern __shared__ int32_t s_d[];
  __shared__ int32_t s_wave[kDiffThreads / 64];
  constexpr int kWaves = kDiffThreads / 64;
  const int wave = threadIdx.x >> 6;
  const int gw = gx + 1, dn = (gx + 1) * (gy + 1);
  for (int e = threadIdx.x; e < dn; e += kDiffThreads) s_d[e] = diff[e];
  __syncthreads();
  for (int y = wave; y < gy; y += kWaves) wave_prefix_lds(s_d + y * gw, gx, 1);
  __syncthreads();
  for (int x = wave; x < gx; x += kWaves) wave_prefix_lds(s_d + x, gy, gw);
  __syncthreads();
  const int nt = gx * gy;
  const int per = (nt + kDiffThreads - 1) / kDiffThreads;
  const int t0 = threadIdx.x * per;
  int32_t local = 0;
  for (int t = t0; t < t0 + per && t < nt; ++t) local += s_d[(t / gx) * gw + t % gx];
  int32_t total;
  int32_t start = block_exclusive_scan(local, &total, s_wave);
  for (int t = t0; t < t0 + per && t < nt; ++t) {
    const int32_t c = s_d[(t / gx) * gw + t % gx];
    ranges[2 * t] = c > 0 ? start : 0;
    ranges[2 * t + 1] = c > 0 ? start + c : 0;
    start += c;
  }
  if (!tile_order) return;
  constexpr int kBins = 256;
  __shared__ int32_t s_bin[kBins];
  for (int i = threadIdx.x; i < kBins; i += kDiffThreads) s_bin[i] = 0;
  __syncthreads();
  for (int t = t0; t < t0 + per && t < nt; ++t)
    atomicAdd(&s_bin[cost_bucket(s_d[(t / gx) * gw + t % gx])], 1);
  __syncthreads();
  if (threadIdx.x < 64) {
    // exclusive scan over the bins from the highest bucket down: lane l
    // owns bins 255-4l .. 252-4l
    const int lane = threadIdx.x;
    int v[4], sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = s_bin[kBins - 1 - 4 * lane - j];
      sum += v[j];
    }
    int inc = sum;
#pragma unroll
    for (int dd = 1; dd < 64; dd <<= 1) {
      const int y = __shfl_up(inc, dd, 64);
      if (lane >= dd) inc += y;
    }
    int run = inc - sum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s_bin[kBins - 1 - 4 * lane - j] = run;
      run += v[j];
    }
  }
  __syncthreads();
  for (int t = t0; t < t0 + per && t < nt; ++t)
    tile_order[atomicAdd(&s_bin[cost_bucket(s_d[(t / gx) * gw + t % gx])], 1)] = t;
}

}  // namespace

size_t scan_scratch_elems(int64_t n) {
  size_t total = 0;
  int64_t m = n;
  while (m > 1) {
    m = (m + kScanTile - 1) / kScanTile;
    total += static_cast<size_t>(m);
  }
  return total + 4;
}


int radix_passes(int end_bit) { return (end_bit + 7) / 8; }

size_t radix_scratch_elems(int64_t n) {
  const int64_t nb = (n + kRadixTile - 1) / kRadixTile;
  const size_t hist = static_cast<size_t>(nb) * kRadixBins;
  return hist + kRadixBins + 4;  // per-(digit, block) counts, digit totals
}

namespace {

// Partitioning of n keys: `sub` tiles of `threads` * kRadixItems keys per
// partition, `np` partitions.  sub stays 1 below 2*kRadixTargetParts tiles
// (every tile its own block) and grows beyond, capped at kRadixMaxSub;
// np <= tiles <= the count of kRadixTile tiles, so the spine fits the
// scratch that radix_scratch_elems sizes for one row per kRadixTile tile.
struct RadixParts {
  int np;
  int sub;
  int threads;  // block size of the passes: kRadixThreads or kRadixThreadsLarge
};

int radix_parts(int64_t n, RadixParts* p) {
  p->threads = n >= kRadixLargeMinKeys ? kRadixThreadsLarge : kRadixThreads;
  const int64_t tile = static_cast<int64_t>(p->threads) * kRadixItems;
  const int64_t tiles = (n + tile - 1) / tile;
  int64_t sub =
      tiles / (p->threads == kRadixThreadsLarge ? kRadixTargetParts : kRadixTargetPartsSmall);
  if (sub < 1) sub = 1;
  if (sub > kRadixMaxSub) sub = kRadixMaxSub;
  const int64_t np = (tiles + sub - 1) / sub;
  if (np > 0x7FFFFFFF) {
    set_error("radix sort: too many keys (%lld)", static_cast<long long>(n));
    return HRF_ERR_INVALID;
  }
  p->np = static_cast<int>(np);
  p->sub = static_cast<int>(sub);
  return HRF_OK;
}

template <int RB, bool VALS>
int radix_pass(const uint32_t* src_k, const uint32_t* src_v, uint32_t* dst_k, uint32_t* dst_v,
               int64_t n, const RadixParts& rp, int shift, uint32_t mask, uint32_t* scratch,
               const uint32_t* run_flag, hipStream_t s, uint32_t out_mask = 0xFFFFFFFFu,
               const SortFirstPass* fp = nullptr, int narrow = -1, uint8_t* tag_out = nullptr) {
  // fp: the histogram is in the scratch already (taken by the pair
  // emission over its blocks, which are this pass's partitions).  narrow
  // >= 0: the pass writes one word per pair into dst_k, the key bits above
  // this digit shifted over the value's `narrow` bits (VALS only).
  // tag_out: each written key's bit 31 as a byte beside it.
  const int nshift = shift + __builtin_popcount(mask);
  const int np = fp ? fp->np : rp.np;
  const int64_t hist_n = static_cast<int64_t>(np) << RB;
  uint32_t* hist = scratch;
  uint32_t* totals = scratch + hist_n;
  const bool large = rp.threads == kRadixThreadsLarge;
  if (!fp) {
    if (large)
      hipLaunchKernelGGL((k_radix_hist<RB, kRadixThreadsLarge>), dim3(rp.np),
                         dim3(kRadixThreadsLarge), 0, s, src_k, n, shift, mask, hist, rp.np,
                         rp.sub, run_flag);
    else
      hipLaunchKernelGGL((k_radix_hist<RB, kRadixThreads>), dim3(rp.np), dim3(kRadixThreads), 0,
                         s, src_k, n, shift, mask, hist, rp.np, rp.sub, run_flag);
    HRF_LAUNCH_CHECK();
  }
  hipLaunchKernelGGL(k_radix_rowscan, dim3(1 << RB), dim3(kRowScanThreads), 0, s, hist, np,
                     totals, run_flag);
  HRF_LAUNCH_CHECK();
  const int64_t* bounds = fp ? fp->bounds : nullptr;
  // With the emission's histogram a scatter block takes fp->group emission
  // blocks (the spine still has one column per emission block).
  const int sub = fp ? fp->group : rp.sub;
  const int nblk = fp ? (np + fp->group - 1) / fp->group : np;
  if (narrow >= 0 && (!VALS || !dst_k)) {
    set_error("internal: a narrowing radix pass needs values and a word output");
    return HRF_ERR_INVALID;
  }
  if (fp && fp->gen) {
    // The emission stored no pair: regenerate and scatter them (one block
    // per emission block).
    const EmitGen& g = *fp->gen;
    if (fp->group != 1 || g.k != n) {
      set_error("internal: fused emission-scatter needs one emission block per partition");
      return HRF_ERR_INVALID;
    }
    if (large)
      hipLaunchKernelGGL((k_emit_scatter<VALS, RB, kRadixThreadsLarge>), dim3(np),
                         dim3(kRadixThreadsLarge), 0, s, g.part_t, g.part_r, g.tiles, g.order,
                         g.sorted_flag, g.rect, g.n, g.k, g.gx, g.vbits, dst_k, dst_v, shift,
                         mask, hist, totals, np, narrow, nshift, g.tags);
    else
      hipLaunchKernelGGL((k_emit_scatter<VALS, RB, kRadixThreads>), dim3(np),
                         dim3(kRadixThreads), 0, s, g.part_t, g.part_r, g.tiles, g.order,
                         g.sorted_flag, g.rect, g.n, g.k, g.gx, g.vbits, dst_k, dst_v, shift,
                         mask, hist, totals, np, narrow, nshift, g.tags);
    HRF_LAUNCH_CHECK();
    return HRF_OK;
  }
  if (large)
    hipLaunchKernelGGL((k_radix_scatter<RB, VALS, kRadixThreadsLarge>), dim3(nblk),
                       dim3(kRadixThreadsLarge), 0, s, src_k, src_v, dst_k, dst_v, n, shift, mask,
                       hist, totals, np, sub, run_flag, out_mask, bounds, narrow, nshift,
                       tag_out);
  else
    hipLaunchKernelGGL((k_radix_scatter<RB, VALS, kRadixThreads>), dim3(nblk),
                       dim3(kRadixThreads), 0, s, src_k, src_v, dst_k, dst_v, n, shift, mask, hist,
                       totals, np, sub, run_flag, out_mask, bounds, narrow, nshift, tag_out);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

// Digit width of pass `pass` of `passes` over nbits key bits: widths differ
// by at most one and the wider digits come last (13 bits: 6 then 7).  The
// first pass moves the most bytes per element (the later ones may write
// less), and fewer digits there mean fewer, longer output runs per tile.
int digit_bits(int nbits, int passes, int pass) {
  const int base = nbits / passes, extra = nbits % passes;
  return base + (pass >= passes - extra ? 1 : 0);
}

// Pass over digit bits [shift, shift + bits) with the narrowest digit
// template that holds them (bits <= 8).
template <bool VALS>
int radix_pass_bits(int bits, const uint32_t* src_k, const uint32_t* src_v, uint32_t* dst_k,
                    uint32_t* dst_v, int64_t n, const RadixParts& rp, int shift,
                    uint32_t* scratch, const uint32_t* run_flag, hipStream_t s,
                    uint32_t out_mask = 0xFFFFFFFFu, const SortFirstPass* fp = nullptr,
                    int narrow = -1, uint8_t* tag_out = nullptr) {
  const uint32_t mask = (1u << bits) - 1u;
  switch (bits) {
    case 1: case 2: case 3: case 4:
      return radix_pass<4, VALS>(src_k, src_v, dst_k, dst_v, n, rp, shift, mask, scratch,
                                 run_flag, s, out_mask, fp, narrow, tag_out);
    case 5:
      return radix_pass<5, VALS>(src_k, src_v, dst_k, dst_v, n, rp, shift, mask, scratch,
                                 run_flag, s, out_mask, fp, narrow, tag_out);
    case 6:
      return radix_pass<6, VALS>(src_k, src_v, dst_k, dst_v, n, rp, shift, mask, scratch,
                                 run_flag, s, out_mask, fp, narrow, tag_out);
    case 7:
      return radix_pass<7, VALS>(src_k, src_v, dst_k, dst_v, n, rp, shift, mask, scratch,
                                 run_flag, s, out_mask, fp, narrow, tag_out);
    case 8:
      return radix_pass<8, VALS>(src_k, src_v, dst_k, dst_v, n, rp, shift, mask, scratch,
                                 run_flag, s, out_mask, fp, narrow, tag_out);
    default:
      set_error("internal: radix digit of %d bits", bits);
      return HRF_ERR_INVALID;
  }
}

}  // namespace

int radix_sort_pairs(uint32_t* ka, uint32_t* va, uint32_t* kb, uint32_t* vb, int64_t n,
                     int end_bit, uint32_t* scratch, bool* result_in_b, hipStream_t s,
                     const uint32_t* run_flag, bool index_values, bool keys_needed,
                     const SortFirstPass* first) {
  *result_in_b = false;
  if (n <= 1) return HRF_OK;
  if (end_bit < 1 || end_bit > 32) {
    set_error("internal: radix sort over %d key bits", end_bit);
    return HRF_ERR_INVALID;
  }
  const int passes = radix_passes(end_bit);
  RadixParts rp{};
  HRF_TRY(radix_parts(n, &rp));
  uint32_t *src_k = ka, *src_v = va, *dst_k = kb, *dst_v = vb;
  int done = 0;
  for (int pass = 0; pass < passes; ++pass) {
    const int bits = digit_bits(end_bit, passes, pass);
    const uint32_t* vin = (pass == 0 && index_values) ? nullptr : src_v;
    uint32_t* kout = (pass == passes - 1 && !keys_needed) ? nullptr : dst_k;
    HRF_TRY(radix_pass_bits<true>(bits, src_k, vin, kout, dst_v, n, rp, done, scratch, run_flag,
                                  s, 0xFFFFFFFFu, pass == 0 ? first : nullptr));
    done += bits;
    uint32_t* tk = src_k;
    uint32_t* tv = src_v;
    src_k = dst_k;
    src_v = dst_v;
    dst_k = tk;
    dst_v = tv;
  }
  *result_in_b = (passes % 2) == 1;
  return HRF_OK;
}

int radix_sort_pairs_narrowed(uint32_t* ka, const uint32_t* va, uint32_t* kb, int64_t n,
                              int end_bit, int vbits, uint32_t* scratch, hipStream_t s,
                              uint32_t* final_out, const SortFirstPass* first,
                              uint8_t* tags) {
  const int passes = radix_passes(end_bit);
  const int bits0 = passes >= 2 ? digit_bits(end_bit, passes, 0) : 0;
  if (n <= 1 || passes < 2 || end_bit > 32 || vbits < 1 ||
      end_bit - bits0 + vbits > (tags ? 31 : 32) || !final_out) {
    set_error("internal: narrowed pair sort of %d key bits over %d value bits", end_bit, vbits);
    return HRF_ERR_INVALID;
  }
  if (tags && !(first && first->gen && first->gen->tags.rec)) {
    set_error("internal: pair tags need the tagging emission-scatter");
    return HRF_ERR_INVALID;
  }
  RadixParts rp{};
  HRF_TRY(radix_parts(n, &rp));
  // Pass 0 on the low digit, writing (key >> bits0) << vbits | value into kb.
  HRF_TRY(radix_pass_bits<true>(bits0, ka, va, kb, nullptr, n, rp, 0, scratch, nullptr, s,
                                0xFFFFFFFFu, first, vbits));
  // The remaining key bits sit at [vbits, vbits + end_bit - bits0) of the
  // words: a key sort whose last pass writes the values into final_out.
  bool in_b = false;
  return radix_sort_keys(kb, ka, n, vbits, end_bit - bits0, scratch, &in_b, s, final_out,
                         (1u << vbits) - 1u, nullptr, tags);
}

int radix_sort_keys(uint32_t* ka, uint32_t* kb, int64_t n, int lo_bit, int nbits,
                    uint32_t* scratch, bool* result_in_b, hipStream_t s, uint32_t* final_out,
                    uint32_t final_mask, const SortFirstPass* first, uint8_t* final_tags) {
  *result_in_b = false;
  if (n <= 1 || nbits <= 0) {
    if (final_out) {
      set_error("internal: radix_sort_keys final output needs n > 1 and nbits > 0");
      return HRF_ERR_INVALID;
    }
    return HRF_OK;
  }
  const int passes = radix_passes(nbits);
  RadixParts rp{};
  HRF_TRY(radix_parts(n, &rp));
  uint32_t *src = ka, *dst = kb;
  int done = 0;
  for (int pass = 0; pass < passes; ++pass) {
    const int bits = digit_bits(nbits, passes, pass);
    const bool last = pass == passes - 1 && final_out;
    uint32_t* out = last ? final_out : dst;
    const uint32_t om = last ? final_mask : 0xFFFFFFFFu;
    HRF_TRY(radix_pass_bits<false>(bits, src, nullptr, out, nullptr, n, rp, lo_bit + done,
                                   scratch, nullptr, s, om, pass == 0 ? first : nullptr, -1,
                                   last ? final_tags : nullptr));
    done += bits;
    uint32_t* t = src;
    src = dst;
    dst = t;
  }
  *result_in_b = !final_out && (passes % 2) == 1;
  return HRF_OK;
}

int launch_fill_u32(uint32_t* p, uint32_t v, int64_t n, hipStream_t s) {
  if (n <= 0) return HRF_OK;
  hipLaunchKernelGGL(k_fill_u32, dim3(blocks_for(n, 256)), dim3(256), 0, s, p, v, n);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_fill_f32(float* p, float v, int64_t n, hipStream_t s) {
  if (n <= 0) return HRF_OK;
  int64_t head = 0;
  if ((reinterpret_cast<uintptr_t>(p) & 15) == 0 && n >= 1024) {
    const int64_t n4 = n / 4;
    hipLaunchKernelGGL(k_fill_f32x4, dim3(blocks_for(n4, 256 * kFillVec)), dim3(256), 0, s,
                       reinterpret_cast<float4*>(p), v, n4);
    HRF_LAUNCH_CHECK();
    head = 4 * n4;
  }
  if (head < n) {
    hipLaunchKernelGGL(k_fill_f32, dim3(blocks_for(n - head, 256)), dim3(256), 0, s, p + head, v,
                       n - head);
    HRF_LAUNCH_CHECK();
  }
  return HRF_OK;
}

int launch_offsets(const uint32_t* order, const uint32_t* tiles, const uint32_t* vis,
                   int64_t n, uint64_t* off, uint32_t* vis_off, uint64_t* bsum_p,
                   uint32_t* bsum_v, const uint32_t* sort_flag, uint64_t* totals,
                   hipStream_t s, uint64_t tag) {
  if (n <= 0) return HRF_OK;
  const int64_t nb = (n + kScanTile - 1) / kScanTile;
  hipLaunchKernelGGL(k_offsets_reduce, dim3(static_cast<unsigned>(nb)), dim3(kScanThreads), 0,
                     s, order, tiles, vis, n, bsum_p, bsum_v);
  HRF_LAUNCH_CHECK();
  hipLaunchKernelGGL((k_offsets_blocks<>), dim3(1), dim3(kScanThreads), 0, s, bsum_p, bsum_v,
                     nb, off + n, sort_flag, totals, nullptr, tag);
  HRF_LAUNCH_CHECK();
  hipLaunchKernelGGL(k_offsets_scan, dim3(static_cast<unsigned>(nb)), dim3(kScanThreads), 0, s,
                     order, tiles, vis, n, bsum_p, bsum_v, off, vis_off);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

namespace {
// Emission blocks grouped into the first pass's scatter partitions: groups
// of at least kFirstPassTargetPairs pairs where that leaves at least
// kFirstPassMinParts partitions; no fused histogram when the groups would
// hold fewer than half that many pairs.
constexpr int64_t kFirstPassTargetPairs = 4 * static_cast<int64_t>(kRadixTile);
constexpr int64_t kFirstPassMinParts = 1024;
int digit_template_bits(int bits) { return bits <= 4 ? 4 : bits; }
// Offset of the partition bounds in the sort scratch: after the spine and
// the digit totals (at most kRadixBins), 8-byte aligned.
int64_t first_bounds_off(int64_t np, int bits) {
  return ((np << digit_template_bits(bits)) + kRadixBins + 1) & ~int64_t(1);
}
EmitHist emit_hist_of(uint32_t* scratch, const SortFirstPass* first, int shift, int bits) {
  if (!first) return EmitHist{nullptr, nullptr, 0, 0u, 0};
  return EmitHist{scratch, const_cast<int64_t*>(first->bounds), shift, (1u << bits) - 1u,
                  1 << digit_template_bits(bits)};
}
}  // namespace

int radix_first_bits(int nbits) { return nbits > 0 ? nbits / radix_passes(nbits) : 0; }

bool emit_first_pass(int64_t n, int64_t k, int bits, uint32_t* scratch, SortFirstPass* first) {
  if (n <= 0 || k <= 1 || bits < 1 || bits > 8 || !scratch) return false;
  const int64_t np = blocks_for(n, kEmitThreads);
  if (np > 0x7FFFFFFF) return false;
  // HRF_SORT_REGENERATE=1 (for tests) takes the fused emission-scatter at
  // any size: one emission block per partition; =2 takes the emission's
  // histogram over groups of its blocks (the stored pairs then scattered by
  // the first pass) at any size.
  const char* force = std::getenv("HRF_SORT_REGENERATE");
  const bool forced = force && force[0] == '1';
  const bool forced_hist = force && force[0] == '2';
  // Below the large sorts the first pass takes tile-aligned partitions of
  // several tiles and its own histogram (headline: emission + first pass
  // 2.8 us faster than with the emission's histogram over its blocks).
  if (!forced && !forced_hist && k < kRadixLargeMinKeys) return false;
  const int64_t avg = k / np > 0 ? k / np : 1;  // pairs per emission block
  int64_t group = (kFirstPassTargetPairs + avg - 1) / avg;
  if (np / group < kFirstPassMinParts) group = np / kFirstPassMinParts;
  if (group < 1 || forced) group = 1;
  if (!forced && !forced_hist && avg * group < kFirstPassTargetPairs / 2) return false;
  const int64_t need = first_bounds_off(np, bits) + 2 * (np + 1);
  if (need > static_cast<int64_t>(radix_scratch_elems(k))) return false;
  first->np = static_cast<int>(np);
  first->bounds = reinterpret_cast<const int64_t*>(scratch + first_bounds_off(np, bits));
  first->group = static_cast<int>(group);
  first->regenerate = group == 1 && (k >= kRadixLargeMinKeys || forced);
  first->gen = nullptr;
  return true;
}

int launch_emit_pairs(const uint64_t* part_t, const uint64_t* part_r, const uint32_t* tiles,
                      const uint32_t* order, const uint32_t* sorted_flag, const uint2* rect,
                      int64_t n, int64_t k, int gx, uint32_t* keys, uint32_t* vals,
                      hipStream_t s, const uint32_t* vis, const uint32_t* part_v,
                      int64_t* visible, int64_t vmax, uint32_t* scratch,
                      const SortFirstPass* first, int first_shift, int first_bits) {
  if (k <= 0 || n <= 0) return HRF_OK;
  const VisibleOut vo{vis, part_v, visible, vmax};
  const EmitHist eh = emit_hist_of(scratch, first, first_shift, first_bits);
  if (eh.hist && first->gen)
    hipLaunchKernelGGL((k_emit_packed<true, true, false>), dim3(blocks_for(n, kEmitThreads)),
                       dim3(kEmitThreads), 0, s, part_t, part_r, tiles, order, sorted_flag, rect,
                       n, k, gx, 0, keys, vals, vo, eh);
  else if (eh.hist)
    hipLaunchKernelGGL((k_emit_packed<true, true>), dim3(blocks_for(n, kEmitThreads)),
                       dim3(kEmitThreads), 0, s, part_t, part_r, tiles, order, sorted_flag, rect,
                       n, k, gx, 0, keys, vals, vo, eh);
  else
    hipLaunchKernelGGL((k_emit_packed<true, false>), dim3(blocks_for(n, kEmitThreads)),
                       dim3(kEmitThreads), 0, s, part_t, part_r, tiles, order, sorted_flag, rect,
                       n, k, gx, 0, keys, vals, vo, eh);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_emit_packed(const uint64_t* part_t, const uint64_t* part_r, const uint32_t* tiles,
                       const uint32_t* order, const uint32_t* sorted_flag, const uint2* rect,
                       int64_t n, int64_t k, int gx, int vbits, uint32_t* words, hipStream_t s,
                       const uint32_t* vis, const uint32_t* part_v, int64_t* visible,
                       int64_t vmax, uint32_t* scratch, const SortFirstPass* first,
                       int first_shift, int first_bits) {
  if (n <= 0) return HRF_OK;
  const VisibleOut vo{vis, part_v, visible, vmax};
  const EmitHist eh = emit_hist_of(scratch, first, first_shift, first_bits);
  if (eh.hist && first->gen)
    hipLaunchKernelGGL((k_emit_packed<false, true, false>), dim3(blocks_for(n, kEmitThreads)),
                       dim3(kEmitThreads), 0, s, part_t, part_r, tiles, order, sorted_flag, rect,
                       n, k, gx, vbits, words, nullptr, vo, eh);
  else if (eh.hist)
    hipLaunchKernelGGL((k_emit_packed<false, true>), dim3(blocks_for(n, kEmitThreads)),
                       dim3(kEmitThreads), 0, s, part_t, part_r, tiles, order, sorted_flag, rect,
                       n, k, gx, vbits, words, nullptr, vo, eh);
  else
    hipLaunchKernelGGL((k_emit_packed<false, false>), dim3(blocks_for(n, kEmitThreads)),
                       dim3(kEmitThreads), 0, s, part_t, part_r, tiles, order, sorted_flag, rect,
                       n, k, gx, vbits, words, nullptr, vo, eh);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int64_t tile_diff_elems(int gx, int gy) {
  return static_cast<int64_t>(gx + 1) * static_cast<int64_t>(gy + 1);
}

bool tile_diff_fits(int gx, int gy) { return tile_diff_elems(gx, gy) <= kMaxTileDiff; }

int launch_tile_ranges_from_rects(const uint32_t* tiles, const uint2* rect, int64_t n, int gx,
                                  int gy, int32_t* diff, int32_t* ranges, hipStream_t s,
                                  int32_t* tile_order) {
  if (!tile_diff_fits(gx, gy)) {
    set_error("internal: tile grid %dx%d too large for the LDS difference array", gx, gy);
    return HRF_ERR_INVALID;
  }
  const int dn = static_cast<int>(tile_diff_elems(gx, gy));
  const size_t lds = static_cast<size_t>(dn) * sizeof(int32_t);
  if (n > 0) {
    const int64_t want = (n + kDiffItems * kDiffThreads - 1) / (kDiffItems * kDiffThreads);
    const int blocks = static_cast<int>(want < kDiffBlocks ? want : kDiffBlocks);
    hipLaunchKernelGGL(k_tile_diff, dim3(blocks), dim3(kDiffThreads), lds, s, tiles, rect, n, gx,
                       dn, diff);
    HRF_LAUNCH_CHECK();
  }
  hipLaunchKernelGGL(k_ranges_from_diff, dim3(1), dim3(kDiffThreads), lds, s, diff, gx, gy,
                     ranges, tile_order);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_unpack_ranges(const uint32_t* words, int64_t k, int vbits, int32_t* point_list,
                         int32_t* ranges, int ntiles, hipStream_t s) {
  HRF_TRY(launch_fill_u32(reinterpret_cast<uint32_t*>(ranges), 0u, 2 * int64_t(ntiles), s));
  if (k <= 0) return HRF_OK;
  hipLaunchKernelGGL(k_unpack_ranges, dim3(blocks_for(k, 256)), dim3(256), 0, s, words, k,
                     vbits, point_list, ranges, static_cast<uint32_t>(ntiles));
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_tile_ranges(const uint32_t* keys, int64_t k, int32_t* ranges, int ntiles,
                       hipStream_t s) {
  HRF_TRY(launch_fill_u32(reinterpret_cast<uint32_t*>(ranges), 0u, 2 * int64_t(ntiles), s));
  if (k <= 0) return HRF_OK;
  hipLaunchKernelGGL(k_tile_ranges, dim3(blocks_for(k, 256)), dim3(256), 0, s, keys, k,
                     ranges, static_cast<uint32_t>(ntiles));
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int64_t partial_elems(int64_t n) { return (n + kProjThreads - 1) / kProjThreads + 1; }

int launch_partials_scan(uint64_t* part_t, uint32_t* part_v, int64_t n, uint32_t* sort_flag,
                         uint64_t* totals, hipStream_t s, uint64_t tag) {
  if (n <= 0) return HRF_OK;
  const int64_t nb = (n + kProjThreads - 1) / kProjThreads;
  hipLaunchKernelGGL((k_offsets_blocks<1024, 4>), dim3(1), dim3(1024), 0, s, part_t, part_v,
                     nb, part_t + nb, nullptr, totals, sort_flag, tag);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

int launch_rank_partials(const uint32_t* order, const uint32_t* tiles, int64_t n,
                         uint64_t* part_r, hipStream_t s) {
  if (n <= 0) return HRF_OK;
  const int64_t nb = (n + kProjThreads - 1) / kProjThreads;
  hipLaunchKernelGGL(k_rank_partials, dim3(static_cast<unsigned>(nb)), dim3(kProjThreads), 0, s,
                     order, tiles, n, part_r);
  HRF_LAUNCH_CHECK();
  hipLaunchKernelGGL((k_offsets_blocks<1024, 4>), dim3(1), dim3(1024), 0, s, part_r, nullptr,
                     nb, part_r + nb, nullptr, nullptr, nullptr, 0ull);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

}  // namespace hrf
