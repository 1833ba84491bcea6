// hrf_internal.h — shared constants, error plumbing, workspace carving and
// device helpers for the gfx950 rasterizer / ASM library.
//
// The whole library is compiled with -ffp-contract=off: every floating-point
// expression that must reproduce the reference bit-for-bit (projection,
// culling, radius, tile rectangles, transfer-function phase) is evaluated in
// source order, and fused multiply-adds are written out with fmaf() only
// where the reference's own arithmetic is a dot product (the cuBLAS matmul
// chain of forward.cu:265-268 / backward.cu:426-439).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "hrf.h"

namespace hrf {

// Compile-time constants of the reference (wave_rasterizer/config.h:15-23).
constexpr int kTile = 16;                     // BLOCK_X == BLOCK_Y
constexpr int kBlock = kTile * kTile;         // threads per render block
// Gaussians per projection block = ranks per emission block = indices per
// visible-compaction block: the granularity of the count partial sums.
constexpr int kProjThreads = 256;
// Bit of a projection block's visible-count partial that carries its
// unsorted-depth flag (the count itself is at most kProjThreads).
constexpr uint32_t kPartFlag = 0x80000000u;
constexpr float kPlaneCutoff = 1e-6f;         // PLANE_PROBABILITY_CUTOFF
constexpr float kMaxAlpha = 0.99f;            // MAX_ALPHA_VALUE
constexpr float kMinAlphaBwd = 1.0f / 255.0f; // backward_splat.cu:218
constexpr float kTermT = 0.0001f;             // forward_splat.cu:243
constexpr int kMaxChannels = 3;               // MAX_CHANNELS
constexpr int kMaxPlanes = 32;                // plane membership is a u32 bitmask

// ---------------------------------------------------------------- errors --
void set_error(const char* fmt, ...);
const char* get_error();

#define HRF_HIP(expr)                                                         \
  do {                                                                        \
    hipError_t e_ = (expr);                                                   \
    if (e_ != hipSuccess) {                                                   \
      ::hrf::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                       __FILE__, __LINE__);                                   \
      return HRF_ERR_HIP;                                                     \
    }                                                                         \
  } while (0)

#define HRF_LAUNCH_CHECK()                                                    \
  do {                                                                        \
    hipError_t e_ = hipGetLastError();                                        \
    if (e_ != hipSuccess) {                                                   \
      ::hrf::set_error("kernel launch failed: %s (%s:%d)",                    \
                       hipGetErrorString(e_), __FILE__, __LINE__);            \
      return HRF_ERR_HIP;                                                     \
    }                                                                         \
  } while (0)

#define HRF_TRY(expr)             \
  do {                            \
    int s_ = (expr);              \
    if (s_ != HRF_OK) return s_;  \
  } while (0)

// -------------------------------------------------------- host read-back --
// Small device results the host must read (pair / visible counts): pinned,
// coherent host words that a kernel writes directly (through `dev`).  Slots
// come from a per-process pool (one slot per concurrent caller and device;
// never freed), so calls on different streams or threads never share one.
struct Readback {
  uint64_t* host;  // 8 words: [0, 3) the counts, [3] the completion tag
  uint64_t* dev;   // the same words as a device address
  int device;
  uint64_t seq;    // tags handed out so far
};
// A free slot of the current device (allocated on first need).
int readback_acquire(Readback** out);
// Sets host[0, 4) to all ones before the writing kernel is queued, so a
// write that is not visible reads as an out-of-range count, never a stale
// one from an earlier call, and returns the tag (never 0 or all ones) the
// kernel must write to host[3] last.
uint64_t readback_arm(Readback* r);
// Waits for the tag (polling the pinned word for a bounded time, then
// synchronising stream s, where the writing kernel was queued) and checks
// it arrived.
int readback_wait(Readback* r, uint64_t tag, hipStream_t s);
void readback_release(Readback* r);
// Holds a slot for one call.  `pending` is set once the writing kernel is
// queued and cleared by a successful wait: a slot left pending (an error
// between the two) is never handed out again, since that kernel may still
// write to it.
struct ReadbackSlot {
  Readback* r = nullptr;
  bool pending = false;
  ReadbackSlot() = default;
  ReadbackSlot(const ReadbackSlot&) = delete;
  ReadbackSlot& operator=(const ReadbackSlot&) = delete;
  ~ReadbackSlot() {
    if (r && !pending) readback_release(r);
  }
};

// ------------------------------------------------------- workspace carving --
// A bump allocator over a caller-provided buffer.  Run once with base ==
// nullptr to size a workspace, then with the real buffer to carve it; both
// runs take the same sequence of requests, so sizes always agree.
struct Carver {
  char* base;
  size_t off = 0;
  explicit Carver(void* b) : base(static_cast<char*>(b)) {}
  template <typename T>
  T* take(size_t count) {
    off = (off + 255) & ~size_t(255);
    T* p = reinterpret_cast<T*>(base ? base + off : nullptr);
    off += count * sizeof(T);
    return p;
  }
  size_t bytes() const { return (off + 255) & ~size_t(255); }
};

// Scope that brackets a stage with hipEvents on its stream while tracing is
// enabled (hrf_trace_enable); a no-op otherwise.
class StageTimer {
 public:
  StageTimer(const char* stage, hipStream_t s);
  ~StageTimer();
  StageTimer(const StageTimer&) = delete;
  StageTimer& operator=(const StageTimer&) = delete;

 private:
  const char* stage_;
  hipStream_t s_;
  hipEvent_t start_ = nullptr, stop_ = nullptr;
  bool active_ = false;
};
#define HRF_CAT2(a, b) a##b
#define HRF_CAT(a, b) HRF_CAT2(a, b)
#define HRF_STAGE(name, s) ::hrf::StageTimer HRF_CAT(hrf_stage_, __LINE__)(name, s)

inline int blocks_for(int64_t n, int per_block) {
  return static_cast<int>((n + per_block - 1) / per_block);
}

// Render record layout, floats: [mx, my, i00, i01, i10, i11, opacity, w,
// amp_re0, amp_im0, ...] padded to a multiple of 4 floats.  Slot 7 is 0 in
// the per-Gaussian array and receives the plane weight when a render block
// stages the record in LDS.
__host__ __device__ constexpr int rec_quads(int channels) {
  return (8 + 2 * channels + 3) / 4;
}
__host__ __device__ constexpr int rec_stride(int channels) {
  return 4 * rec_quads(channels);
}
// Per-Gaussian backward accumulator: [dmx, dmy, dcov_xx, dcov_xy,
// dcov_yy, A_0..A_{C-1}, B_0..B_{C-1}, Q_0..Q_{P-1}].
__host__ __device__ constexpr int acc_stride(int channels, int planes) {
  return 5 + 2 * channels + planes;
}

// ------------------------------------------------------ launch interfaces --
struct ProjectParams {
  const float* cam;
  const float* z;
  const float* quats;
  const float* scales;
  const float* colours;
  const float* phase;
  const float* opac;
  const float* pprobs;
  const float* view;
  int64_t n;
  int C, P;
  float fx, fy, px, py;
  float lim_x, lim_y;  // 1.3 * half tan fov (host-evaluated as the reference)
  int W, H, gx, gy;
  float near_plane, far_plane;
  // outputs
  float* rec;       // n * rec_stride(C)
  uint32_t* pmask;  // n
  uint2* rect;      // n: x = minx | miny << 16, y = maxx | maxy << 16
  uint32_t* tiles;  // n
  uint32_t* dkey;   // n: depth sort key
  uint32_t* vis;    // n: 0/1
  // optional: per kProjThreads-block sums of tiles (u64) and vis (u32); bit
  // kPartFlag of part_v is set when some depth key of the block is below its
  // predecessor's
  uint64_t* part_t;
  uint32_t* part_v;
  // optional: cleared by the launch (the tile difference array that a later
  // kernel of the same call accumulates into)
  int32_t* zero;
  int64_t zero_n;
};
int launch_project(const ProjectParams& p, hipStream_t s);

struct GeomBwdParams {
  const float* cam;
  const float* z;
  const float* quats;
  const float* scales;
  const float* colours;
  const float* phase;
  const float* opac;
  const float* pprobs;
  const float* view;
  const float* acc;  // n * acc_stride(C,P)
  int64_t n;
  int C, P;
  float fx, fy;
  float lim_x, lim_y;
  float near_plane, far_plane;
  float* g_cam;
  float* g_z;
  float* g_quat;
  float* g_scale;
  float* g_col;
  float* g_phase;
  float* g_opac;
  float* g_plane;
};
int launch_geom_backward(const GeomBwdParams& p, hipStream_t s);

// Scan scratch sizing (block-sum pyramid of an n-element scan).
size_t scan_scratch_elems(int64_t n);

// Stable LSD radix sort of (u32 key, u32 value) pairs over bits
// [0, end_bit).  Ping-pongs between (ka,va) and (kb,vb); returns in
// *result_in_b whether the sorted data ended in (kb,vb).  With run_flag, the
// passes do nothing on the device while *run_flag == 0 (callers use an even
// pass count then, so the data stays in (ka,va) either way).
size_t radix_scratch_elems(int64_t n);
// ceil(end_bit/8) passes, digit widths differing by at most one (the wider
// ones last).  With index_values, the values are taken to be 0..n-1 (va is
// only used as a buffer).  keys_needed == false: the last pass writes only
// the values (the sorted keys are then left nowhere).
// A first sort pass whose histogram the pair emission took: np emission
// blocks, block b's pairs being [bounds[b], bounds[b + 1]), their counts
// already in the sort scratch (digit-major, np columns).  The pass's
// scatter partitions are `group` consecutive emission blocks each.
// Inputs of the pair tags (render_cull.h): the render records, their stride
// and the plane weights (n x P).  rec == nullptr: no tags.
struct TagSrc {
  const float* rec;
  int rec_stride;
  const float* pprobs;
  int P;
};
// What the fused emission-scatter needs to regenerate the emission's pairs
// (the emission launch's own inputs), and with tags.rec set (wide keys
// only), what it needs to tag each pair in value bit 31 with the forward's
// visibility test (pair_visible).
struct EmitGen {
  const uint64_t* part_t;
  const uint64_t* part_r;
  const uint32_t* tiles;
  const uint32_t* order;
  const uint32_t* sorted_flag;
  const uint2* rect;
  int64_t n;
  int64_t k;
  int gx;
  int vbits;
  TagSrc tags;
};
// regenerate (set by emit_first_pass): the sort is large enough (8192-key
// tiles, one emission block per partition) for the emission to store no
// pair and the first pass to regenerate them from `gen`, which the caller
// sets (nullptr: the emission stores the pairs and the pass reads them).
struct SortFirstPass {
  int np;
  const int64_t* bounds;
  int group;
  bool regenerate;
  const EmitGen* gen;
};
int radix_sort_pairs(uint32_t* ka, uint32_t* va, uint32_t* kb, uint32_t* vb,
                     int64_t n, int end_bit, uint32_t* scratch, bool* result_in_b,
                     hipStream_t s, const uint32_t* run_flag = nullptr,
                     bool index_values = false, bool keys_needed = true,
                     const SortFirstPass* first = nullptr);
int radix_passes(int end_bit);
// Stable sort of (key, value) pairs on key bits [0, end_bit) (two or more
// passes) that keeps one word per pair after the first pass: that pass
// writes (key >> d0) << vbits | value into kb (d0 its digit bits; needs
// end_bit - d0 + vbits <= 32 and values below 2^vbits), and the later
// passes sort those words on bits [vbits, vbits + end_bit - d0) as
// radix_sort_keys, the last writing the values into final_out.  Four bytes
// move per pair in the later passes instead of eight.  ka and kb are
// overwritten; first: as for radix_sort_pairs.  tags != nullptr: the
// fused emission-scatter tags the pairs (first->gen->tags set; needs
// end_bit - d0 + vbits <= 31, the tag riding in word bit 31 through the
// later passes) and the last pass writes each pair's tag (0 or 1) into
// tags[i] beside final_out[i].
int radix_sort_pairs_narrowed(uint32_t* ka, const uint32_t* va, uint32_t* kb, int64_t n,
                              int end_bit, int vbits, uint32_t* scratch, hipStream_t s,
                              uint32_t* final_out, const SortFirstPass* first = nullptr,
                              uint8_t* tags = nullptr);
// Whether radix_sort_pairs_narrowed applies to end_bit key bits and vbits
// value bits (spare = 1: with a tag bit beside them).
inline bool narrowed_sort_fits(int end_bit, int vbits, int spare = 0) {
  const int passes = radix_passes(end_bit);
  if (passes < 2 || end_bit > 32) return false;
  const int d0 = end_bit / passes;  // the first pass's digit (the narrowest)
  return end_bit - d0 + vbits + spare <= 32;
}
// Stable LSD radix sort of u32 words on bits [lo_bit, lo_bit + nbits) only
// (the other bits ride along unsorted), in ceil(nbits/8) passes with the
// digit widths of radix_sort_pairs; same scratch and ping-pong convention.
// final_out != nullptr (needs n > 1, nbits > 0): the last pass writes
// word & final_mask there instead of into the ping-pong buffers, and with
// final_tags, word >> 31 into final_tags (one byte per word).
int radix_sort_keys(uint32_t* ka, uint32_t* kb, int64_t n, int lo_bit, int nbits,
                    uint32_t* scratch, bool* result_in_b, hipStream_t s,
                    uint32_t* final_out = nullptr, uint32_t final_mask = 0xFFFFFFFFu,
                    const SortFirstPass* first = nullptr, uint8_t* final_tags = nullptr);
// Whether the pair emission of n Gaussians and k pairs takes the first
// tile-sort pass's histogram (of `bits` digit bits): only when groups of
// consecutive emission blocks hold several sort tiles of pairs each while
// enough groups remain to fill the GPU (with ~1-2 tiles per partition the
// partial tiles would cost the scatter what the histogram saves), and the
// spine and partition bounds fit `scratch` (radix scratch for k keys).
// Fills *first (its bounds inside the scratch, the group size) when so.
bool emit_first_pass(int64_t n, int64_t k, int bits, uint32_t* scratch, SortFirstPass* first);
// Digit bits of the first pass of a sort over nbits bits (the narrowest).
int radix_first_bits(int nbits);

// Tile ranges from the Gaussians' tile rectangles (tiles[g] > 0 marks a
// rectangle) instead of the sorted pairs: a 2-D difference array of
// (gx+1)(gy+1) int32 in `diff` (device scratch that must hold zeros: the
// projection of the same call clears it), integrated in one block.
// Only for tile grids whose difference array fits kMaxTileDiff entries.
constexpr int64_t kMaxTileDiff = 16000;  // 64000 B of LDS
// Cost bucket of a list length: 8 buckets per octave of (c + 1), 256 in
// all (the render kernels' longest-first block orders).
__device__ __forceinline__ int cost_bucket(int c) {
  const unsigned v = static_cast<unsigned>(c < 0 ? 0 : c) + 1u;
  const int e = 31 - __clz(v);
  const unsigned mant = e >= 3 ? (v >> (e - 3)) & 7u : (v << (3 - e)) & 7u;
  return e * 8 + static_cast<int>(mant);
}
int64_t tile_diff_elems(int gx, int gy);
bool tile_diff_fits(int gx, int gy);
int launch_tile_ranges_from_rects(const uint32_t* tiles, const uint2* rect, int64_t n, int gx,
                                  int gy, int32_t* diff, int32_t* ranges, hipStream_t s,
                                  int32_t* tile_order = nullptr);

// Exclusive pair offsets off[0..n] (off[n] = K) of the tile counts taken in
// depth-rank order (tiles[order[i]]; order == nullptr: index order) and
// exclusive visible offsets vis_off (index order); totals receives
// [K, V, *sort_flag] and, when tag != 0, totals[3] = tag after a
// system-scope fence (the host polls it).  bsum_p / bsum_v: ceil(n / 2048) elements each.
int launch_offsets(const uint32_t* order, const uint32_t* tiles, const uint32_t* vis,
                   int64_t n, uint64_t* off, uint32_t* vis_off, uint64_t* bsum_p,
                   uint32_t* bsum_v, const uint32_t* sort_flag, uint64_t* totals,
                   hipStream_t s, uint64_t tag = 0);
// Count partials: part_t / part_v hold per-kProjThreads-block sums (from
// k_project, index order, part_v with the kPartFlag bits); launch_partials_scan
// turns them, in place, into exclusive block bases (part_t[nb] = K), writes
// the OR of the flags to *sort_flag and totals [K, V, flag].
// launch_rank_partials forms part_r, the same for the tile counts taken in
// depth-rank order (tiles[order[r]]), and scans it (totals untouched).
int launch_partials_scan(uint64_t* part_t, uint32_t* part_v, int64_t n, uint32_t* sort_flag,
                         uint64_t* totals, hipStream_t s, uint64_t tag = 0);
int launch_rank_partials(const uint32_t* order, const uint32_t* tiles, int64_t n,
                         uint64_t* part_r, hipStream_t s);
// The emit kernels take the scanned bases: part_t (index order) or, when
// *sorted_flag, part_r (rank order), and form each block's pair offsets
// from the tile counts themselves; the depth-order permutation they use is
// order[] when *sorted_flag != 0 and the identity otherwise.  With
// `visible`, the emit launch also writes the visible compaction (the
// indices with vis set, in order: index block b of 256 from vis and the
// scanned bases part_v; same grid as the emission).
int launch_emit_pairs(const uint64_t* part_t, const uint64_t* part_r, const uint32_t* tiles,
                      const uint32_t* order, const uint32_t* sorted_flag, const uint2* rect,
                      int64_t n, int64_t k, int gx, uint32_t* keys, uint32_t* vals,
                      hipStream_t s, const uint32_t* vis = nullptr,
                      const uint32_t* part_v = nullptr, int64_t* visible = nullptr,
                      int64_t vmax = 0, uint32_t* scratch = nullptr,
                      const SortFirstPass* first = nullptr, int first_shift = 0,
                      int first_bits = 0);
// (first->gen set: the emission only counts the first pass's digits and
// stores no pair; the sort's first pass regenerates them.)
int launch_tile_ranges(const uint32_t* keys, int64_t k, int32_t* ranges,
                       int ntiles, hipStream_t s);
// Packed binning (tile bits + gaussian bits <= 32): word = tile << vbits | g.
int launch_emit_packed(const uint64_t* part_t, const uint64_t* part_r, const uint32_t* tiles,
                       const uint32_t* order, const uint32_t* sorted_flag, const uint2* rect,
                       int64_t n, int64_t k, int gx, int vbits, uint32_t* words, hipStream_t s,
                       const uint32_t* vis = nullptr, const uint32_t* part_v = nullptr,
                       int64_t* visible = nullptr, int64_t vmax = 0,
                       uint32_t* scratch = nullptr, const SortFirstPass* first = nullptr,
                       int first_shift = 0, int first_bits = 0);
int launch_unpack_ranges(const uint32_t* words, int64_t k, int vbits, int32_t* point_list,
                         int32_t* ranges, int ntiles, hipStream_t s);
int64_t partial_elems(int64_t n);  // kProjThreads-blocks + 1
int launch_fill_u32(uint32_t* p, uint32_t v, int64_t n, hipStream_t s);
int launch_fill_f32(float* p, float v, int64_t n, hipStream_t s);

struct RenderParams {
  const int32_t* ranges;
  const int32_t* plist;
  // Forward, optional: tile ids longest list first (tile_order_n of them);
  // the blocks then take the tiles in that order, a tile's planes on one
  // XCD.
  const int32_t* tile_order;
  int tile_order_n;
  // Optional pair tags beside plist (large wide-key sorts): 0 marks an entry
  // the forward culls in every plane (render_cull.h, pair_visible), which
  // the forward then skips without gathering its plane mask or record.
  const uint8_t* ptag;
  const uint32_t* pmask;
  const float* rec;
  const float* pprobs;
  int64_t n;          // Gaussians: list entries outside [0, n) are skipped
  int64_t num_pairs;  // list length: ranges are clamped to [0, num_pairs]
  int C, P, W, H, gx, gy;
  // forward outputs
  float2* field;
  float* final_T;
  int32_t* n_contrib;
  // backward inputs / outputs
  const float2* grad_field;
  const float* final_T_in;
  const int32_t* n_contrib_in;
  float* acc;
  // Plane member lists (optional).  Entry i of (tile t, plane q) is the
  // (gaussian, tile-list position) pair of the i-th member of plane q in
  // t's list, stored at q*num_pairs + r0(t) + i; sub_cnt[t*P + q] members.
  // The forward writes them (sub_out) for the batches it composites; the
  // backward then reads them (sub) instead of re-filtering every tile list
  // per plane.
  int2* sub_out;
  int32_t* sub_cnt_out;
  const int2* sub;
  const int32_t* sub_cnt;
  // Backward block order over the T*P (tile, plane) ids (with sub): longest
  // member list first.
  const int32_t* order;
  // Forward, optional: the plane-0 block of each tile copies its ranges
  // entry here (ranges formed in a workspace reach the caller's array).
  int32_t* ranges_out;
};
int launch_render_forward(const RenderParams& p, hipStream_t s);
int launch_render_empty(const RenderParams& p, hipStream_t s);
int launch_render_backward(const RenderParams& p, hipStream_t s);
// Backward prologue, one launch: acc[0, n) = 0 and, when order != nullptr
// and m > 0, order[0..m) = the ids 0..m-1 sorted by cnt[id] descending (in
// logarithmic buckets, 8 per octave; arbitrary order inside a bucket).
int launch_bwd_prologue(float* acc, int64_t n, const int32_t* cnt, int m, int32_t* order,
                        hipStream_t s);

// ASM (band-limited angular spectrum).
struct AsmConsts {
  float k;        // (float)(2*pi/(double)lambda)
  float fx_max;   // band limit along rows
  float fy_max;   // band limit along cols
  float dist;     // signed distance used in the phase
  int pass;       // fx_max/fy_max computed; always 1
};
AsmConsts asm_consts(float wavelength, float distance, float pixel_pitch, int nx, int ny);

int launch_asm_spectral_grid(const float* re, const float* im, const float* fxg,
                             const float* fyg, float* ore, float* oim, int nx, int ny,
                             float wavelength, float distance, float aperture,
                             float pitch, bool adjoint, hipStream_t s);
int launch_asm_pad(const float2* in, int batch, int h, int w, float2* out, int M,
                   hipStream_t s);
int launch_asm_crop(const float2* in, int batch, int M, int h, int w, float scale,
                    float2* out, hipStream_t s);
int launch_asm_mac_forward(const float2* spec, int P, int C, int M, double pitch,
                           const float* wavelengths, const float* distances,
                           float aperture, float2* out, hipStream_t s);
int launch_asm_mac_adjoint(const float2* spec, int P, int C, int M, double pitch,
                           const float* wavelengths, const float* distances,
                           float aperture, float2* out, hipStream_t s);
// One distance of a multi-distance propagation over C channel spectra:
// out[c] (+)= spec[c] * T(wavelengths[c], distance) * A, conj(T) for adjoint.
int launch_asm_mac_distance(const float2* spec, int C, int M, double pitch,
                            const float* wavelengths, float distance, float aperture,
                            bool adjoint, bool accumulate, float2* out, hipStream_t s);
int fft_c2c(float2* buf, int M, int batch, bool inverse, hipStream_t s);
void fft_release_all();

// Fused LDS-FFT propagation (asm_fft.hip) for the grid sizes it has plans
// for.  X needs P*C*H*M (forward) / C*S*M (adjoint) complex elements, Z
// C*S*M / P*C*H*M.
bool fused_fft_supported(int M);
int fused_asm_forward(const float2* fields, int P, int C, int H, int W, int S, double pitch,
                      const float* wl, const float* dist, float ap, float2* holo, float2* X,
                      float2* Z, hipStream_t s);
int fused_asm_adjoint(const float2* gholo, int P, int C, int H, int W, int S, double pitch,
                      const float* wl, const float* dist, float ap, float2* gfields, float2* X,
                      float2* Z, hipStream_t s);
// Multi-distance forward (C,H,W) -> (D,C,S,S) and adjoint (D,C,S,S) ->
// (C,H,W), `group` distances per column pass.  Forward: X needs C*H*M and Z
// group*C*S*M elements; adjoint: X group*C*S*M and Z C*H*M.
int fused_md_forward(const float2* field, int D, int C, int H, int W, int S, double pitch,
                     const float* wl, const float* dist, float ap, float2* out, float2* X,
                     float2* Z, int group, hipStream_t s);
int fused_md_adjoint(const float2* gout, int D, int C, int H, int W, int S, double pitch,
                     const float* wl, const float* dist, float ap, float2* gfield, float2* X,
                     float2* Z, int group, hipStream_t s);
void fused_fft_release_all();

}  // namespace hrf
