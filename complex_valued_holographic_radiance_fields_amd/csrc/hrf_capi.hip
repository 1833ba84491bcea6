// hrf_capi.hip — extern "C" entry points declared in include/hrf.h.
//
// Host-side orchestration only: argument validation, workspace carving,
// launch sequencing on the caller's stream.  The only allocations are the
// pinned read-back slots for the count read-backs (64 bytes and an event
// each, a few per device, kept until the process ends) and, in the ASM file,
// hipFFT's plan work areas (cached per device/size).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <atomic>
#include <chrono>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "hrf_internal.h"

namespace hrf {

namespace {
thread_local std::string g_err;
}

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
}

const char* get_error() { return g_err.c_str(); }

namespace {
std::mutex g_rb_mu;
std::vector<Readback*> g_rb_free;
}  // namespace

int readback_acquire(Readback** out) {
  int dev = 0;
  HRF_HIP(hipGetDevice(&dev));
  {
    std::lock_guard<std::mutex> lk(g_rb_mu);
    for (size_t i = 0; i < g_rb_free.size(); ++i) {
      if (g_rb_free[i]->device == dev) {
        *out = g_rb_free[i];
        g_rb_free.erase(g_rb_free.begin() + static_cast<std::ptrdiff_t>(i));
        return HRF_OK;
      }
    }
  }
  Readback r{nullptr, nullptr, dev, 0};
  HRF_HIP(hipHostMalloc(reinterpret_cast<void**>(&r.host), 8 * sizeof(uint64_t),
                        hipHostMallocCoherent | hipHostMallocMapped));
  HRF_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&r.dev), r.host, 0));
  *out = new Readback(r);
  return HRF_OK;
}

uint64_t readback_arm(Readback* r) {
  volatile uint64_t* h = r->host;
  for (int i = 0; i < 4; ++i) h[i] = ~0ull;
  std::atomic_thread_fence(std::memory_order_seq_cst);
  r->seq = r->seq + 1 >= ~0ull - 1 ? 1 : r->seq + 1;
  return r->seq;
}

int readback_wait(Readback* r, uint64_t tag, hipStream_t s) {
  // A stream or event wait can take tens of microseconds to return after
  // the GPU signals; polling the tag word sees the kernel's last write within
  // about a microsecond.  The poll is bounded: past the bound a stream
  // synchronisation (which returns once everything queued has run) takes
  // over.
  // HRF_READBACK_SPIN_US overrides the bound (0: always the stream wait).
  auto spin = std::chrono::microseconds(20000);
  if (const char* e = std::getenv("HRF_READBACK_SPIN_US")) spin = std::chrono::microseconds(std::atoll(e));
  const volatile uint64_t* h = r->host;
  const auto t0 = std::chrono::steady_clock::now();
  bool seen = false;
  if (spin.count() > 0) {
    for (int i = 0;; ++i) {
      if (h[3] == tag) {
        seen = true;
        break;
      }
      if ((i & 255) == 255 && std::chrono::steady_clock::now() - t0 > spin) break;
      __builtin_ia32_pause();
    }
  }
  if (!seen) {
    HRF_HIP(hipStreamSynchronize(s));
    if (h[3] != tag) {
      set_error("internal: count read-back tag %llu not seen after the stream (read %llu)",
                static_cast<unsigned long long>(tag), static_cast<unsigned long long>(h[3]));
      return HRF_ERR_HIP;
    }
  }
  std::atomic_thread_fence(std::memory_order_acquire);
  return HRF_OK;
}

void readback_release(Readback* r) {
  std::lock_guard<std::mutex> lk(g_rb_mu);
  g_rb_free.push_back(r);
}

namespace {
// The counts hrf_raster_forward_prepare returned, per geometry workspace
// (the last prepare on each), so hrf_raster_forward_render can reject counts
// that differ from them before anything is enqueued.  Bounded: past
// kMaxPrepared workspaces the oldest record is dropped (the render then has
// only the kernels' own output bounds to rely on).
struct Prepared {
  const void* ws;
  int64_t n, k, v;
};
constexpr size_t kMaxPrepared = 256;
std::mutex g_prep_mu;
std::vector<Prepared> g_prep;
}  // namespace

void prepared_record(const void* ws, int64_t n, int64_t k, int64_t v) {
  std::lock_guard<std::mutex> lk(g_prep_mu);
  for (auto& e : g_prep) {
    if (e.ws == ws) {
      e = Prepared{ws, n, k, v};
      return;
    }
  }
  if (g_prep.size() >= kMaxPrepared) g_prep.erase(g_prep.begin());
  g_prep.push_back(Prepared{ws, n, k, v});
}

int prepared_check(const void* ws, int64_t n, int64_t k, int64_t v) {
  std::lock_guard<std::mutex> lk(g_prep_mu);
  for (const auto& e : g_prep) {
    if (e.ws != ws) continue;
    if (e.n != n || e.k != k || e.v != v) {
      set_error("forward render: counts (N %lld, K %lld, V %lld) differ from what "
                "hrf_raster_forward_prepare returned for this geometry workspace "
                "(N %lld, K %lld, V %lld)",
                static_cast<long long>(n), static_cast<long long>(k),
                static_cast<long long>(v), static_cast<long long>(e.n),
                static_cast<long long>(e.k), static_cast<long long>(e.v));
      return HRF_ERR_INVALID;
    }
    return HRF_OK;
  }
  return HRF_OK;
}

namespace {

// Backward workspaces whose prologue (accumulator clear + block order)
// hrf_raster_backward_prepare has queued: the workspace, what it was
// prepared for, and an event recorded after the prologue on the preparing
// stream.  hrf_raster_backward on a matching record waits for the event
// instead of running the prologue, and consumes the record.
struct BwdPrepared {
  const void* ws;
  int64_t n, num_pairs;
  int C, P;
  const void* plane_lists;
  hipEvent_t done;
  bool armed;
};
constexpr size_t kMaxBwdPrepared = 64;
std::mutex g_bprep_mu;
std::vector<BwdPrepared> g_bprep;

// ------------------------------------------------------------ validation --
int check_raster_args(const hrf_gaussians* g, const hrf_camera* cam) {
  if (!g || !cam) {
    set_error("null gaussians/camera descriptor");
    return HRF_ERR_INVALID;
  }
  if (g->n < 0 || g->n > 0x7FFFFFFFLL) {
    set_error("number of Gaussians must be in [0, 2^31) (got %lld)",
              static_cast<long long>(g->n));
    return HRF_ERR_INVALID;
  }
  if (g->channels < 1 || g->channels > kMaxChannels) {
    set_error("number of channels must be 1..%d (got %d); the reference supports at most "
              "MAX_CHANNELS=3",
              kMaxChannels, g->channels);
    return HRF_ERR_INVALID;
  }
  if (g->planes < 1 || g->planes > kMaxPlanes) {
    set_error("number of planes must be 1..%d (got %d)", kMaxPlanes, g->planes);
    return HRF_ERR_INVALID;
  }
  if (cam->width <= 0 || cam->height <= 0) {
    set_error("image size must be positive (got %dx%d)", cam->width, cam->height);
    return HRF_ERR_INVALID;
  }
  const int gx = (cam->width + kTile - 1) / kTile, gy = (cam->height + kTile - 1) / kTile;
  if (gx > 65535 || gy > 65535 || static_cast<int64_t>(gx) * gy * g->planes > 0x7FFFFFFFLL) {
    set_error("image too large (%dx%d)", cam->width, cam->height);
    return HRF_ERR_INVALID;
  }
  if (g->n > 0 && (!g->cam_means || !g->z_vals || !g->quats || !g->scales || !g->colours ||
                   !g->phase || !g->opacities || !g->plane_probs || !cam->view_matrix)) {
    set_error("null input pointer");
    return HRF_ERR_INVALID;
  }
  return HRF_OK;
}

struct Frame {
  int gx, gy, ntiles;
  float lim_x, lim_y;
};

Frame frame_of(const hrf_camera* cam) {
  Frame f;
  f.gx = (cam->width + kTile - 1) / kTile;
  f.gy = (cam->height + kTile - 1) / kTile;
  f.ntiles = f.gx * f.gy;
  // half_tan_fov = 0.5f * width / fx (forward.cu:199-200), lim = 1.3f * it.
  const float htx = 0.5f * static_cast<float>(cam->width) / cam->fx;
  const float hty = 0.5f * static_cast<float>(cam->height) / cam->fy;
  f.lim_x = 1.3f * htx;
  f.lim_y = 1.3f * hty;
  return f;
}

// ------------------------------------------------------ geometry workspace --
struct GeomWs {
  float* rec;
  uint32_t* pmask;
  uint2* rect;
  uint32_t* tiles;
  uint32_t* dkey;
  uint32_t* dkey_b;
  uint32_t* order;
  uint32_t* order_b;
  uint32_t* vis;
  uint64_t* part_t;  // per-projection-block tile sums -> pair bases (index order)
  uint32_t* part_v;  // per-projection-block visible sums -> visible bases
  uint64_t* part_r;  // pair bases in depth-rank order (when the depth sort runs)
  uint32_t* radix;
  uint32_t* sort_flag;
  // Tile ranges formed in the prepare call when the tile grid's difference
  // array fits kMaxTileDiff (the render call then reads them here).
  int32_t* diff;
  int32_t* ranges;
  int32_t* tile_order;  // tile ids, longest list first (the forward's block order)
};

GeomWs carve_geom(Carver& cv, int64_t n, int C) {
  GeomWs w;
  const int64_t m = n > 0 ? n : 1;
  w.rec = cv.take<float>(static_cast<size_t>(m) * rec_stride(C));
  w.pmask = cv.take<uint32_t>(m);
  w.rect = cv.take<uint2>(m);
  w.tiles = cv.take<uint32_t>(m);
  w.dkey = cv.take<uint32_t>(m);
  w.dkey_b = cv.take<uint32_t>(m);
  w.order = cv.take<uint32_t>(m);
  w.order_b = cv.take<uint32_t>(m);

  w.vis = cv.take<uint32_t>(m);
  w.part_t = cv.take<uint64_t>(partial_elems(m));
  w.part_v = cv.take<uint32_t>(partial_elems(m));
  w.part_r = cv.take<uint64_t>(partial_elems(m));
  w.radix = cv.take<uint32_t>(radix_scratch_elems(m));
  w.sort_flag = cv.take<uint32_t>(4);
  w.diff = cv.take<int32_t>(kMaxTileDiff);
  w.ranges = cv.take<int32_t>(2 * kMaxTileDiff);
  w.tile_order = cv.take<int32_t>(kMaxTileDiff);
  return w;
}

struct BinWs {
  uint32_t* keys_a;
  uint32_t* keys_b;
  uint32_t* vals_s;
  uint32_t* radix;
};

BinWs carve_bin(Carver& cv, int64_t k) {
  BinWs w;
  const int64_t m = k > 0 ? k : 1;
  w.keys_a = cv.take<uint32_t>(m);
  w.keys_b = cv.take<uint32_t>(m);
  w.vals_s = cv.take<uint32_t>(m);
  w.radix = cv.take<uint32_t>(radix_scratch_elems(m));
  return w;
}

// Plane member lists: P*K (gaussian, position) entries, T*P counts, and the
// backward's block order over the T*P (tile, plane) ids.
struct SubWs {
  int2* entries;
  int32_t* counts;
  int32_t* order;
};

SubWs carve_sub(Carver& cv, int64_t k, int ntiles, int P) {
  SubWs w;
  const int64_t m = k > 0 ? k : 1;
  const size_t tp = static_cast<size_t>(ntiles > 0 ? ntiles : 1) * (P > 0 ? P : 1);
  w.entries = cv.take<int2>(static_cast<size_t>(m) * (P > 0 ? P : 1));
  w.counts = cv.take<int32_t>(tp);
  w.order = cv.take<int32_t>(tp);
  return w;
}

struct BwdWs {
  float* rec;
  uint32_t* pmask;
  uint2* rect;
  uint32_t* tiles;
  uint32_t* dkey;
  uint32_t* vis;
  float* acc;
};

BwdWs carve_bwd(Carver& cv, int64_t n, int C, int P) {
  BwdWs w;
  const int64_t m = n > 0 ? n : 1;
  w.rec = cv.take<float>(static_cast<size_t>(m) * rec_stride(C));
  w.pmask = cv.take<uint32_t>(m);
  w.rect = cv.take<uint2>(m);
  w.tiles = cv.take<uint32_t>(m);
  w.dkey = cv.take<uint32_t>(m);
  w.vis = cv.take<uint32_t>(m);
  w.acc = cv.take<float>(static_cast<size_t>(m) * acc_stride(C, P));
  return w;
}

ProjectParams project_params(const hrf_gaussians* g, const hrf_camera* cam, const Frame& f) {
  ProjectParams p{};
  p.cam = g->cam_means;
  p.z = g->z_vals;
  p.quats = g->quats;
  p.scales = g->scales;
  p.colours = g->colours;
  p.phase = g->phase;
  p.opac = g->opacities;
  p.pprobs = g->plane_probs;
  p.view = cam->view_matrix;
  p.n = g->n;
  p.C = g->channels;
  p.P = g->planes;
  p.fx = cam->fx;
  p.fy = cam->fy;
  p.px = cam->px;
  p.py = cam->py;
  p.lim_x = f.lim_x;
  p.lim_y = f.lim_y;
  p.W = cam->width;
  p.H = cam->height;
  p.gx = f.gx;
  p.gy = f.gy;
  p.near_plane = cam->near_plane;
  p.far_plane = cam->far_plane;
  return p;
}

int bits_for(int ntiles) {
  int b = 0;
  while (b < 31 && (1u << b) < static_cast<uint32_t>(ntiles)) ++b;
  return b;
}

// Pair counts index the reference's int32 point_list / ranges outputs
// (rasterizer_splat.cu:430 holds the count in an int).
int check_pair_count(int64_t k) {
  if (k < 0) {
    set_error("invalid pair count %lld", static_cast<long long>(k));
    return HRF_ERR_INVALID;
  }
  if (k > 0x7FFFFFFFLL) {
    set_error("pair count %lld exceeds the int32 point_list/ranges format",
              static_cast<long long>(k));
    return HRF_ERR_OVERFLOW;
  }
  return HRF_OK;
}

int check_ws(void* ws, size_t have, size_t need, const char* what) {
  if (need > 0 && (!ws || have < need)) {
    set_error("%s workspace too small: %zu bytes given, %zu needed", what, have, need);
    return HRF_ERR_WORKSPACE;
  }
  return HRF_OK;
}

int check_asm(int P, int C, int H, int W, int S) {
  if (P < 1 || P > kMaxPlanes || C < 1 || C > kMaxChannels) {
    set_error("asm: planes must be 1..%d and channels 1..%d (got %d, %d)", kMaxPlanes,
              kMaxChannels, P, C);
    return HRF_ERR_INVALID;
  }
  if (S <= 0 || H <= 0 || W <= 0 || H > 2 * S || W > 2 * S) {
    set_error("asm: field %dx%d does not fit the padded grid 2*%d", H, W, S);
    return HRF_ERR_INVALID;
  }
  if ((H & 1) || (W & 1) || (S & 1)) {
    set_error("asm: sizes must be even (field %dx%d, size %d): centred pad/crop of odd sizes "
              "is ill-defined in the reference (odak crop_center returns size-1)",
              H, W, S);
    return HRF_ERR_INVALID;
  }
  if (static_cast<int64_t>(2 * S) * (2 * S) > 0x7FFFFFFFLL) {
    set_error("asm: grid too large (size %d)", S);
    return HRF_ERR_INVALID;
  }
  return HRF_OK;
}

}  // namespace
}  // namespace hrf

using namespace hrf;

extern "C" {

const char* hrf_last_error(void) { return hrf::get_error(); }

const char* hrf_version(void) { return "hrf 0.1 gfx950"; }

size_t hrf_raster_geom_workspace_size(int64_t n, int32_t channels, int32_t planes) {
  (void)planes;
  Carver cv(nullptr);
  carve_geom(cv, n, channels < 1 ? 1 : (channels > 3 ? 3 : channels));
  return cv.bytes();
}

size_t hrf_raster_binning_workspace_size(int64_t num_pairs, int32_t width, int32_t height) {
  if (num_pairs < 0 || width <= 0 || height <= 0) return 0;
  Carver cv(nullptr);
  carve_bin(cv, num_pairs);
  return cv.bytes();
}

size_t hrf_raster_plane_lists_size(int64_t num_pairs, int32_t width, int32_t height,
                                   int32_t planes) {
  if (num_pairs < 0 || width <= 0 || height <= 0 || planes <= 0) return 0;
  const int ntiles = ((width + kTile - 1) / kTile) * ((height + kTile - 1) / kTile);
  Carver cv(nullptr);
  carve_sub(cv, num_pairs, ntiles, planes);
  return cv.bytes();
}

size_t hrf_raster_backward_workspace_size(int64_t n, int32_t channels, int32_t planes) {
  Carver cv(nullptr);
  carve_bwd(cv, n, channels < 1 ? 1 : (channels > 3 ? 3 : channels),
            planes < 1 ? 1 : planes);
  return cv.bytes();
}

int hrf_raster_forward_prepare(const hrf_gaussians* g, const hrf_camera* cam, void* geom_ws,
                               size_t geom_ws_bytes, void* stream, int64_t* num_pairs,
                               int64_t* num_visible) {
  HRF_TRY(check_raster_args(g, cam));
  if (!num_pairs || !num_visible) {
    set_error("null count outputs");
    return HRF_ERR_INVALID;
  }
  *num_pairs = 0;
  *num_visible = 0;
  const int64_t n = g->n;
  if (n == 0) return HRF_OK;
  HRF_TRY(check_ws(geom_ws, geom_ws_bytes,
                   hrf_raster_geom_workspace_size(n, g->channels, g->planes), "geometry"));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const Frame f = frame_of(cam);
  Carver cv(geom_ws);
  GeomWs w = carve_geom(cv, n, g->channels);

  ProjectParams pp = project_params(g, cam, f);
  pp.rec = w.rec;
  pp.pmask = w.pmask;
  pp.rect = w.rect;
  pp.tiles = w.tiles;
  pp.dkey = w.dkey;
  pp.vis = w.vis;
  pp.part_t = w.part_t;
  pp.part_v = w.part_v;
  const bool diff_ranges = tile_diff_fits(f.gx, f.gy);
  if (diff_ranges) {
    pp.zero = w.diff;
    pp.zero_n = tile_diff_elems(f.gx, f.gy);
  }
  ReadbackSlot slot;
  HRF_TRY(readback_acquire(&slot.r));
  const uint64_t tag = readback_arm(slot.r);
  {
    HRF_STAGE("project", s);
    HRF_TRY(launch_project(pp, s));
  }

  // K and V from the projection's per-block sums (index order: K and V do
  // not depend on the order, and the reference's caller hands Gaussians over
  // already sorted by depth, Scene.render, model.py:1387, where index order
  // is depth order); the sums become the blocks' pair / visible bases.  The
  // scan writes [K, V, flag] straight into the pinned read-back words.
  {
    HRF_STAGE("scan", s);
    slot.pending = true;
    HRF_TRY(launch_partials_scan(w.part_t, w.part_v, n, w.sort_flag, slot.r->dev, s, tag));
  }
  // The tile ranges need only the rectangles: they run while the host waits
  // for the counts (and the render call reads them from the workspace).
  if (diff_ranges) {
    HRF_STAGE("ranges", s);
    HRF_TRY(launch_tile_ranges_from_rects(w.tiles, w.rect, n, f.gx, f.gy, w.diff, w.ranges, s,
                                          w.tile_order));
  }
  HRF_TRY(readback_wait(slot.r, tag, s));
  slot.pending = false;
  const uint64_t host_tot[3] = {slot.r->host[0], slot.r->host[1], slot.r->host[2]};
  if (host_tot[1] > static_cast<uint64_t>(n) || host_tot[2] > 1) {
    set_error("internal: count read-back incomplete (V %llu, flag %llu)",
              static_cast<unsigned long long>(host_tot[1]),
              static_cast<unsigned long long>(host_tot[2]));
    return HRF_ERR_INVALID;
  }
  if (host_tot[0] > 0x7FFFFFFFull) {
    set_error("pair count %llu exceeds the int32 point_list/ranges format",
              static_cast<unsigned long long>(host_tot[0]));
    return HRF_ERR_OVERFLOW;
  }
  if (host_tot[2] != 0) {
    // k_project found a depth key below its predecessor's: stable depth
    // ordering of the Gaussians (32-bit keys, 4 passes: the sorted order
    // ends in the first buffer pair), then the pair offsets in that order.
    {
      HRF_STAGE("depth_sort", s);
      bool in_b = false;
      HRF_TRY(radix_sort_pairs(w.dkey, w.order, w.dkey_b, w.order_b, n, 32, w.radix, &in_b, s,
                               nullptr, true));
      if (in_b) {
        set_error("internal: depth sort expected an even pass count");
        return HRF_ERR_INVALID;
      }
    }
    HRF_STAGE("scan", s);
    HRF_TRY(launch_rank_partials(w.order, w.tiles, n, w.part_r, s));
  }
  *num_pairs = static_cast<int64_t>(host_tot[0]);
  *num_visible = static_cast<int64_t>(host_tot[1]);
  prepared_record(geom_ws, n, *num_pairs, *num_visible);
  return HRF_OK;
}

int hrf_raster_forward_render(const hrf_gaussians* g, const hrf_camera* cam, void* geom_ws,
                              size_t geom_ws_bytes, void* bin_ws, size_t bin_ws_bytes,
                              int64_t num_pairs, int64_t num_visible, void* field,
                              float* final_T, int32_t* n_contrib, int32_t* point_list,
                              int32_t* ranges, int64_t* visible, void* plane_lists,
                              size_t plane_lists_bytes, void* stream) {
  HRF_TRY(check_raster_args(g, cam));
  HRF_TRY(check_pair_count(num_pairs));
  if (num_visible < 0 || num_visible > g->n) {
    set_error("invalid visible count %lld for %lld Gaussians",
              static_cast<long long>(num_visible), static_cast<long long>(g->n));
    return HRF_ERR_INVALID;
  }
  if (!field || !final_T || !n_contrib || !ranges) {
    set_error("null output pointer");
    return HRF_ERR_INVALID;
  }
  if (g->n > 0) HRF_TRY(prepared_check(geom_ws, g->n, num_pairs, num_visible));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const Frame f = frame_of(cam);
  RenderParams rp{};
  rp.C = g->channels;
  rp.P = g->planes;
  rp.W = cam->width;
  rp.H = cam->height;
  rp.gx = f.gx;
  rp.gy = f.gy;
  rp.field = static_cast<float2*>(field);
  rp.final_T = final_T;
  rp.n_contrib = n_contrib;
  if (num_pairs == 0) {
    HRF_TRY(launch_render_empty(rp, s));
    HRF_TRY(launch_fill_u32(reinterpret_cast<uint32_t*>(ranges), 0u, 2 * int64_t(f.ntiles), s));
    return HRF_OK;
  }
  if (!point_list || (num_visible > 0 && !visible)) {
    set_error("null point_list/visible output");
    return HRF_ERR_INVALID;
  }
  const int64_t n = g->n;
  HRF_TRY(check_ws(geom_ws, geom_ws_bytes,
                   hrf_raster_geom_workspace_size(n, g->channels, g->planes), "geometry"));
  HRF_TRY(check_ws(bin_ws, bin_ws_bytes,
                   hrf_raster_binning_workspace_size(num_pairs, cam->width, cam->height),
                   "binning"));
  Carver cg(geom_ws);
  GeomWs w = carve_geom(cg, n, g->channels);
  Carver cb(bin_ws);
  BinWs b = carve_bin(cb, num_pairs);

  // Pair emission in depth-rank order, then a stable sort on the tile id.
  const int end_bit = bits_for(f.ntiles);
  int vbits = bits_for(static_cast<int>(n < 0x7FFFFFFF ? n : 0x7FFFFFFF));
  // HRF_SORT_VBITS=b (for tests): at least b gaussian bits, which takes the
  // two-word key path (and with HRF_SORT_REGENERATE=1 its pair tags) at
  // sizes where one word would hold tile and gaussian.
  if (const char* e = std::getenv("HRF_SORT_VBITS")) {
    const int want = std::atoi(e);
    if (want > vbits && want <= 31) vbits = want;
  }
  // Usual case: the prepare call formed the tile ranges from the Gaussians'
  // rectangles in the geometry workspace (no pass over the sorted pairs);
  // the forward render copies them into `ranges`.
  const bool diff_ranges = tile_diff_fits(f.gx, f.gy);
  // Large pair counts per Gaussian block: the emission also takes the first
  // sort pass's histogram over its blocks.
  SortFirstPass first{};
  const int first_bits = radix_first_bits(end_bit);  // 0 without tile bits (one tile)
  const bool first_fused =
      first_bits > 0 && emit_first_pass(n, num_pairs, first_bits, b.radix, &first);
  // Large sorts of two or more passes: the emission only counts, and the
  // first pass regenerates the pairs (one write of them instead of a
  // write, a read and a write).
  EmitGen gen{w.part_t, w.part_r, w.tiles, w.order, w.sort_flag, w.rect,
              n, num_pairs, f.gx, vbits, TagSrc{}};
  if (first_fused && first.regenerate && radix_passes(end_bit) >= 2) first.gen = &gen;
  // Pair tags for the forward (wide keys whose first pass regenerates the
  // pairs, with a spare word bit after it): the emission-scatter tests each
  // (tile, gaussian) pair as the forward's visibility cull would and the
  // last pass writes the result beside point_list (into the values buffer,
  // free by then), so the forward skips the culled entries of its lists
  // without gathering their records.
  uint8_t* pair_tags = nullptr;
  if (end_bit + vbits > 32 && first.gen && diff_ranges && num_pairs > 1 &&
      narrowed_sort_fits(end_bit, vbits, 1)) {
    gen.tags = TagSrc{w.rec, rec_stride(g->channels), g->plane_probs, g->planes};
    pair_tags = reinterpret_cast<uint8_t*>(b.vals_s);
  }
  if (end_bit + vbits <= 32) {
    // Tile and gaussian fit one word: sort 4-byte words on the tile bits.
    {
      HRF_STAGE("emit", s);
      HRF_TRY(launch_emit_packed(w.part_t, w.part_r, w.tiles, w.order, w.sort_flag, w.rect, n,
                                 num_pairs, f.gx, vbits, b.keys_a, s, w.vis, w.part_v,
                                 num_visible > 0 ? visible : nullptr, num_visible, b.radix,
                                 first_fused ? &first : nullptr, vbits, first_bits));
    }
    bool in_b = false;
    // The last sort pass writes the gaussian bits straight into point_list;
    // otherwise the sorted words are unpacked.  A one-tile image has no
    // tile bits to sort (end_bit 0): the emitted depth-rank order is already
    // the sorted order and the unpack writes it.
    const bool fused = num_pairs > 1 && diff_ranges && end_bit > 0;
    {
      HRF_STAGE("tile_sort", s);
      HRF_TRY(radix_sort_keys(b.keys_a, b.keys_b, num_pairs, vbits, end_bit, b.radix, &in_b, s,
                              fused ? reinterpret_cast<uint32_t*>(point_list) : nullptr,
                              (1u << vbits) - 1u, first_fused ? &first : nullptr));
    }
    if (!fused) {
      HRF_STAGE("ranges", s);
      HRF_TRY(launch_unpack_ranges(in_b ? b.keys_b : b.keys_a, num_pairs, vbits, point_list,
                                   ranges, f.ntiles, s));
    }
  } else if (diff_ranges && num_pairs > 1 && narrowed_sort_fits(end_bit, vbits)) {
    // Tile and gaussian need two words, but after the first sort pass the
    // remaining tile bits and the gaussian fit one: that pass writes packed
    // words and the later ones sort them as the packed path does (4 bytes
    // per pair read and written after the first pass instead of 8).
    {
      HRF_STAGE("emit", s);
      HRF_TRY(launch_emit_pairs(w.part_t, w.part_r, w.tiles, w.order, w.sort_flag, w.rect, n,
                                num_pairs, f.gx, b.keys_a, b.vals_s, s, w.vis, w.part_v,
                                num_visible > 0 ? visible : nullptr, num_visible, b.radix,
                                first_fused ? &first : nullptr, 0, first_bits));
    }
    {
      HRF_STAGE("tile_sort", s);
      HRF_TRY(radix_sort_pairs_narrowed(b.keys_a, b.vals_s, b.keys_b, num_pairs, end_bit, vbits,
                                        b.radix, s, reinterpret_cast<uint32_t*>(point_list),
                                        first_fused ? &first : nullptr, pair_tags));
    }
  } else {
    const bool odd = (radix_passes(end_bit) % 2) == 1;
    uint32_t* vals_a = odd ? b.vals_s : reinterpret_cast<uint32_t*>(point_list);
    uint32_t* vals_b = odd ? reinterpret_cast<uint32_t*>(point_list) : b.vals_s;
    {
      HRF_STAGE("emit", s);
      HRF_TRY(launch_emit_pairs(w.part_t, w.part_r, w.tiles, w.order, w.sort_flag, w.rect, n,
                                num_pairs, f.gx, b.keys_a, vals_a, s, w.vis, w.part_v,
                                num_visible > 0 ? visible : nullptr, num_visible, b.radix,
                                first_fused ? &first : nullptr, 0, first_bits));
    }
    bool in_b = false;
    {
      HRF_STAGE("tile_sort", s);
      // The sorted tile ids are only needed to form the ranges from them.
      HRF_TRY(radix_sort_pairs(b.keys_a, vals_a, b.keys_b, vals_b, num_pairs, end_bit, b.radix,
                               &in_b, s, nullptr, false, !diff_ranges,
                               first_fused ? &first : nullptr));
    }
    const uint32_t* sorted_keys = in_b ? b.keys_b : b.keys_a;
    // The sorted values must end in point_list whatever the pass count did
    // (a single pair is never moved by the sort).
    const uint32_t* sorted_vals = in_b ? vals_b : vals_a;
    if (sorted_vals != reinterpret_cast<uint32_t*>(point_list))
      HRF_HIP(hipMemcpyAsync(point_list, sorted_vals, num_pairs * sizeof(uint32_t),
                             hipMemcpyDeviceToDevice, s));
    if (!diff_ranges) {
      HRF_STAGE("ranges", s);
      HRF_TRY(launch_tile_ranges(sorted_keys, num_pairs, ranges, f.ntiles, s));
    }
  }

  rp.ranges = diff_ranges ? w.ranges : ranges;
  rp.ranges_out = diff_ranges ? ranges : nullptr;
  // Longest tile lists first (formed with the ranges in the prepare call).
  rp.tile_order = diff_ranges ? w.tile_order : nullptr;
  rp.tile_order_n = f.ntiles;
  rp.plist = point_list;
  rp.ptag = pair_tags;
  rp.pmask = w.pmask;
  rp.rec = w.rec;
  rp.pprobs = g->plane_probs;
  rp.n = n;
  rp.num_pairs = num_pairs;
  if (plane_lists) {
    if (n >= (int64_t{1} << 28)) {
      set_error("plane member lists need fewer than 2^28 Gaussians (got %lld)",
                static_cast<long long>(n));
      return HRF_ERR_INVALID;
    }
    HRF_TRY(check_ws(plane_lists, plane_lists_bytes,
                     hrf_raster_plane_lists_size(num_pairs, cam->width, cam->height, g->planes),
                     "plane lists"));
    Carver cs(plane_lists);
    const SubWs sw = carve_sub(cs, num_pairs, f.ntiles, g->planes);
    rp.sub_out = sw.entries;
    rp.sub_cnt_out = sw.counts;
  }
  {
    HRF_STAGE("render_fwd", s);
    HRF_TRY(launch_render_forward(rp, s));
  }
  return HRF_OK;
}

int hrf_raster_backward_prepare(const hrf_gaussians* g, const hrf_camera* cam,
                                int64_t num_pairs, void* ws, size_t ws_bytes, void* plane_lists,
                                size_t plane_lists_bytes, void* stream) {
  HRF_TRY(check_raster_args(g, cam));
  const int64_t n = g->n;
  if (n == 0) return HRF_OK;
  HRF_TRY(check_pair_count(num_pairs));
  HRF_TRY(check_ws(ws, ws_bytes, hrf_raster_backward_workspace_size(n, g->channels, g->planes),
                   "backward"));
  const bool use_sub = plane_lists && num_pairs > 0;
  if (use_sub && n >= (int64_t{1} << 28)) {
    set_error("plane member lists need fewer than 2^28 Gaussians (got %lld)",
              static_cast<long long>(n));
    return HRF_ERR_INVALID;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const Frame f = frame_of(cam);
  Carver cv(ws);
  BwdWs w = carve_bwd(cv, n, g->channels, g->planes);
  SubWs sw{};
  if (use_sub) {
    HRF_TRY(check_ws(plane_lists, plane_lists_bytes,
                     hrf_raster_plane_lists_size(num_pairs, cam->width, cam->height, g->planes),
                     "plane lists"));
    Carver cs(plane_lists);
    sw = carve_sub(cs, num_pairs, f.ntiles, g->planes);
  }
  std::lock_guard<std::mutex> lk(g_bprep_mu);
  BwdPrepared* rec = nullptr;
  for (auto& e : g_bprep)
    if (e.ws == ws) rec = &e;
  if (!rec) {
    if (g_bprep.size() >= kMaxBwdPrepared) {
      set_error("backward prepare: more than %d workspaces prepared at once",
                static_cast<int>(kMaxBwdPrepared));
      return HRF_ERR_INVALID;
    }
    hipEvent_t ev = nullptr;
    HRF_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    g_bprep.push_back(BwdPrepared{ws, 0, 0, 0, 0, nullptr, ev, false});
    rec = &g_bprep.back();
  }
  {
    HRF_STAGE("bwd_prologue", s);
    HRF_TRY(launch_bwd_prologue(w.acc, n * acc_stride(g->channels, g->planes), sw.counts,
                                use_sub ? f.ntiles * g->planes : 0, sw.order, s));
  }
  HRF_HIP(hipEventRecord(rec->done, s));
  rec->n = n;
  rec->num_pairs = num_pairs;
  rec->C = g->channels;
  rec->P = g->planes;
  rec->plane_lists = use_sub ? plane_lists : nullptr;
  rec->armed = true;
  return HRF_OK;
}

int hrf_raster_backward(const hrf_gaussians* g, const hrf_camera* cam, const void* grad_field,
                        const float* final_T, const int32_t* n_contrib,
                        const int32_t* point_list, const int32_t* ranges, int64_t num_pairs,
                        void* ws, size_t ws_bytes, const void* fwd_geom_ws,
                        size_t fwd_geom_ws_bytes, void* plane_lists,
                        size_t plane_lists_bytes, float* grad_cam, float* grad_z,
                        float* grad_quats, float* grad_scales, float* grad_colours,
                        float* grad_phase, float* grad_opacities, float* grad_plane_probs,
                        void* stream) {
  HRF_TRY(check_raster_args(g, cam));
  const int64_t n = g->n;
  if (n == 0) return HRF_OK;
  if (!grad_cam || !grad_z || !grad_quats || !grad_scales || !grad_colours || !grad_phase ||
      !grad_opacities || !grad_plane_probs) {
    set_error("null gradient output pointer");
    return HRF_ERR_INVALID;
  }
  HRF_TRY(check_pair_count(num_pairs));
  if (num_pairs > 0 && (!grad_field || !final_T || !n_contrib || !point_list || !ranges)) {
    set_error("null forward-state pointer");
    return HRF_ERR_INVALID;
  }
  HRF_TRY(check_ws(ws, ws_bytes, hrf_raster_backward_workspace_size(n, g->channels, g->planes),
                   "backward"));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const Frame f = frame_of(cam);
  Carver cv(ws);
  BwdWs w = carve_bwd(cv, n, g->channels, g->planes);

  // Render records: those the forward saved in its geometry workspace (the
  // same inputs give the same records), else recomputed here.
  const float* rec = w.rec;
  const uint32_t* pmask = w.pmask;
  if (fwd_geom_ws) {
    HRF_TRY(check_ws(const_cast<void*>(fwd_geom_ws), fwd_geom_ws_bytes,
                     hrf_raster_geom_workspace_size(n, g->channels, g->planes),
                     "forward geometry"));
    Carver cg(const_cast<void*>(fwd_geom_ws));
    const GeomWs fw = carve_geom(cg, n, g->channels);
    rec = fw.rec;
    pmask = fw.pmask;
  }
  // Plane member lists from the forward: the render backward walks them, in
  // the block order the prologue forms from their counts (written into the
  // lists' order words).
  SubWs sw{};
  const bool use_sub = plane_lists && num_pairs > 0;
  if (use_sub && n >= (int64_t{1} << 28)) {
    set_error("plane member lists need fewer than 2^28 Gaussians (got %lld)",
              static_cast<long long>(n));
    return HRF_ERR_INVALID;
  }
  if (use_sub) {
    HRF_TRY(check_ws(plane_lists, plane_lists_bytes,
                     hrf_raster_plane_lists_size(num_pairs, cam->width, cam->height, g->planes),
                     "plane lists"));
    Carver cs(plane_lists);
    sw = carve_sub(cs, num_pairs, f.ntiles, g->planes);
  }
  {
    HRF_STAGE("project", s);
    if (!fwd_geom_ws) {
      ProjectParams pp = project_params(g, cam, f);
      pp.rec = w.rec;
      pp.pmask = w.pmask;
      pp.rect = w.rect;
      pp.tiles = w.tiles;
      pp.dkey = w.dkey;
      pp.vis = w.vis;
      HRF_TRY(launch_project(pp, s));
    }
    // A prologue that hrf_raster_backward_prepare queued for this same
    // workspace and configuration: wait for it instead.
    bool prepared = false;
    {
      std::lock_guard<std::mutex> lk(g_bprep_mu);
      for (auto& e : g_bprep) {
        if (e.ws != ws || !e.armed) continue;
        e.armed = false;  // consumed (or stale): this call decides
        if (e.n == n && e.num_pairs == num_pairs && e.C == g->channels && e.P == g->planes &&
            e.plane_lists == (use_sub ? plane_lists : nullptr)) {
          HRF_HIP(hipStreamWaitEvent(s, e.done, 0));
          prepared = true;
        }
        break;
      }
    }
    if (!prepared)
      HRF_TRY(launch_bwd_prologue(w.acc, n * acc_stride(g->channels, g->planes), sw.counts,
                                  use_sub ? f.ntiles * g->planes : 0, sw.order, s));
  }

  if (num_pairs > 0) {
    RenderParams rp{};
    rp.ranges = ranges;
    rp.plist = point_list;
    rp.pmask = pmask;
    rp.rec = rec;
    rp.pprobs = g->plane_probs;
    rp.n = n;
    rp.num_pairs = num_pairs;
    rp.C = g->channels;
    rp.P = g->planes;
    rp.W = cam->width;
    rp.H = cam->height;
    rp.gx = f.gx;
    rp.gy = f.gy;
    rp.grad_field = static_cast<const float2*>(grad_field);
    rp.final_T_in = final_T;
    rp.n_contrib_in = n_contrib;
    rp.acc = w.acc;
    if (use_sub) {
      rp.sub = sw.entries;
      rp.sub_cnt = sw.counts;
      rp.order = sw.order;
    }
    HRF_STAGE("render_bwd", s);
    HRF_TRY(launch_render_backward(rp, s));
  }

  GeomBwdParams gb{};
  gb.cam = g->cam_means;
  gb.z = g->z_vals;
  gb.quats = g->quats;
  gb.scales = g->scales;
  gb.colours = g->colours;
  gb.phase = g->phase;
  gb.opac = g->opacities;
  gb.pprobs = g->plane_probs;
  gb.view = cam->view_matrix;
  gb.acc = w.acc;
  gb.n = n;
  gb.C = g->channels;
  gb.P = g->planes;
  gb.fx = cam->fx;
  gb.fy = cam->fy;
  gb.lim_x = f.lim_x;
  gb.lim_y = f.lim_y;
  gb.near_plane = cam->near_plane;
  gb.far_plane = cam->far_plane;
  gb.g_cam = grad_cam;
  gb.g_z = grad_z;
  gb.g_quat = grad_quats;
  gb.g_scale = grad_scales;
  gb.g_col = grad_colours;
  gb.g_phase = grad_phase;
  gb.g_opac = grad_opacities;
  gb.g_plane = grad_plane_probs;
  {
    HRF_STAGE("geom_bwd", s);
    HRF_TRY(launch_geom_backward(gb, s));
  }
  return HRF_OK;
}

// ------------------------------------------------------------------ ASM --

int hrf_asm_spectral_forward(const float* re, const float* im, const float* fx_grid,
                             const float* fy_grid, float* out_re, float* out_im, int32_t nx,
                             int32_t ny, float wavelength, float distance, float aperture,
                             float pixel_pitch, void* stream) {
  if (nx <= 0 || ny <= 0 || nx != ny) {
    set_error("asm spectral: only square grids are defined (got %dx%d)", nx, ny);
    return HRF_ERR_INVALID;
  }
  if (!re || !im || !fx_grid || !fy_grid || !out_re || !out_im) {
    set_error("asm spectral: null pointer");
    return HRF_ERR_INVALID;
  }
  return launch_asm_spectral_grid(re, im, fx_grid, fy_grid, out_re, out_im, nx, ny,
                                  wavelength, distance, aperture, pixel_pitch, false,
                                  static_cast<hipStream_t>(stream));
}

int hrf_asm_spectral_backward(const float* grad_re, const float* grad_im,
                              const float* field_re, const float* field_im,
                              const float* fx_grid, const float* fy_grid, float* out_re,
                              float* out_im, int32_t nx, int32_t ny, float wavelength,
                              float distance, float aperture, float pixel_pitch,
                              void* stream) {
  (void)field_re;
  (void)field_im;
  if (nx <= 0 || ny <= 0 || nx != ny) {
    set_error("asm spectral: only square grids are defined (got %dx%d)", nx, ny);
    return HRF_ERR_INVALID;
  }
  if (!grad_re || !grad_im || !fx_grid || !fy_grid || !out_re || !out_im) {
    set_error("asm spectral: null pointer");
    return HRF_ERR_INVALID;
  }
  return launch_asm_spectral_grid(grad_re, grad_im, fx_grid, fy_grid, out_re, out_im, nx, ny,
                                  wavelength, distance, aperture, pixel_pitch, true,
                                  static_cast<hipStream_t>(stream));
}

size_t hrf_asm_workspace_size(int32_t planes, int32_t channels, int32_t size) {
  if (planes < 1 || channels < 1 || size < 1) return 0;
  const int64_t M = 2 * static_cast<int64_t>(size);
  Carver cv(nullptr);
  cv.take<float2>(static_cast<size_t>(planes) * channels * M * M);
  cv.take<float2>(static_cast<size_t>(channels) * M * M);
  return cv.bytes();
}

int hrf_asm_multiplane_forward(const void* fields, int32_t planes, int32_t channels,
                               int32_t height, int32_t width, int32_t size,
                               const float* wavelengths, const float* distances,
                               double pixel_pitch, float aperture, void* hologram, void* ws,
                               size_t ws_bytes, void* stream) {
  HRF_TRY(check_asm(planes, channels, height, width, size));
  if (!fields || !wavelengths || !distances || !hologram) {
    set_error("asm: null pointer");
    return HRF_ERR_INVALID;
  }
  HRF_TRY(check_ws(ws, ws_bytes, hrf_asm_workspace_size(planes, channels, size), "asm"));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int M = 2 * size;
  const int64_t MM = static_cast<int64_t>(M) * M;
  Carver cv(ws);
  float2* spec = cv.take<float2>(static_cast<size_t>(planes) * channels * MM);
  float2* outs = cv.take<float2>(static_cast<size_t>(channels) * MM);
  const int PC = planes * channels;
  if (fused_fft_supported(M)) {
    return fused_asm_forward(static_cast<const float2*>(fields), planes, channels, height,
                             width, size, pixel_pitch, wavelengths, distances, aperture,
                             static_cast<float2*>(hologram), spec, outs, s);
  }
  {
    HRF_STAGE("asm_pad", s);
    HRF_TRY(launch_asm_pad(static_cast<const float2*>(fields), PC, height, width, spec, M, s));
  }
  {
    HRF_STAGE("asm_fft", s);
    HRF_TRY(fft_c2c(spec, M, PC, false, s));
  }
  {
    HRF_STAGE("asm_mac_fwd", s);
    HRF_TRY(launch_asm_mac_forward(spec, planes, channels, M, pixel_pitch, wavelengths,
                                   distances, aperture, outs, s));
  }
  {
    HRF_STAGE("asm_fft", s);
    HRF_TRY(fft_c2c(outs, M, channels, true, s));
  }
  {
    HRF_STAGE("asm_crop", s);
    HRF_TRY(launch_asm_crop(outs, channels, M, size, size,
                            static_cast<float>(1.0 / static_cast<double>(MM)),
                            static_cast<float2*>(hologram), s));
  }
  return HRF_OK;
}

int hrf_asm_multiplane_adjoint(const void* grad_hologram, int32_t planes, int32_t channels,
                               int32_t height, int32_t width, int32_t size,
                               const float* wavelengths, const float* distances,
                               double pixel_pitch, float aperture, void* grad_fields, void* ws,
                               size_t ws_bytes, void* stream) {
  HRF_TRY(check_asm(planes, channels, height, width, size));
  if (!grad_hologram || !wavelengths || !distances || !grad_fields) {
    set_error("asm: null pointer");
    return HRF_ERR_INVALID;
  }
  HRF_TRY(check_ws(ws, ws_bytes, hrf_asm_workspace_size(planes, channels, size), "asm"));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int M = 2 * size;
  const int64_t MM = static_cast<int64_t>(M) * M;
  Carver cv(ws);
  float2* spec = cv.take<float2>(static_cast<size_t>(planes) * channels * MM);
  float2* gsp = cv.take<float2>(static_cast<size_t>(channels) * MM);
  const int PC = planes * channels;
  if (fused_fft_supported(M)) {
    return fused_asm_adjoint(static_cast<const float2*>(grad_hologram), planes, channels,
                             height, width, size, pixel_pitch, wavelengths, distances, aperture,
                             static_cast<float2*>(grad_fields), gsp, spec, s);
  }
  {
    HRF_STAGE("asm_pad", s);
    HRF_TRY(launch_asm_pad(static_cast<const float2*>(grad_hologram), channels, size, size,
                           gsp, M, s));
  }
  {
    HRF_STAGE("asm_fft", s);
    HRF_TRY(fft_c2c(gsp, M, channels, false, s));
  }
  {
    HRF_STAGE("asm_mac_adj", s);
    HRF_TRY(launch_asm_mac_adjoint(gsp, planes, channels, M, pixel_pitch, wavelengths,
                                   distances, aperture, spec, s));
  }
  {
    HRF_STAGE("asm_fft", s);
    HRF_TRY(fft_c2c(spec, M, PC, true, s));
  }
  {
    HRF_STAGE("asm_crop", s);
    HRF_TRY(launch_asm_crop(spec, PC, M, height, width,
                            static_cast<float>(1.0 / static_cast<double>(MM)),
                            static_cast<float2*>(grad_fields), s));
  }
  return HRF_OK;
}

size_t hrf_asm_multidistance_workspace_size(int32_t channels, int32_t size) {
  if (channels < 1 || size < 1) return 0;
  const int64_t M = 2 * static_cast<int64_t>(size);
  Carver cv(nullptr);
  cv.take<float2>(static_cast<size_t>(channels) * M * M);
  cv.take<float2>(static_cast<size_t>(channels) * M * M);
  return cv.bytes();
}

int hrf_asm_multidistance_forward(const void* field, int32_t num_distances, int32_t channels,
                                  int32_t height, int32_t width, int32_t size,
                                  const float* wavelengths, const float* distances,
                                  double pixel_pitch, float aperture, void* out, void* ws,
                                  size_t ws_bytes, void* stream) {
  HRF_TRY(check_asm(1, channels, height, width, size));
  if (num_distances < 1 || !field || !wavelengths || !distances || !out) {
    set_error("asm multi-distance: null pointer or no distance");
    return HRF_ERR_INVALID;
  }
  HRF_TRY(check_ws(ws, ws_bytes, hrf_asm_multidistance_workspace_size(channels, size),
                   "asm multi-distance"));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int M = 2 * size;
  const int64_t MM = static_cast<int64_t>(M) * M;
  const int64_t SS = static_cast<int64_t>(size) * size;
  Carver cv(ws);
  float2* spec = cv.take<float2>(static_cast<size_t>(channels) * MM);
  float2* buf = cv.take<float2>(static_cast<size_t>(channels) * MM);
  if (fused_fft_supported(M)) {
    // X = spec holds the C row spectra (H <= M rows); buf holds the column
    // results of M / size = 2 distances at a time (C * size * M each).
    return fused_md_forward(static_cast<const float2*>(field), num_distances, channels, height,
                            width, size, pixel_pitch, wavelengths, distances, aperture,
                            static_cast<float2*>(out), spec, buf, M / size, s);
  }
  // The C channel spectra are computed once and shared by every distance.
  {
    HRF_STAGE("asm_pad", s);
    HRF_TRY(launch_asm_pad(static_cast<const float2*>(field), channels, height, width, spec, M,
                           s));
  }
  {
    HRF_STAGE("asm_fft", s);
    HRF_TRY(fft_c2c(spec, M, channels, false, s));
  }
  for (int d = 0; d < num_distances; ++d) {
    {
      HRF_STAGE("asm_mac_fwd", s);
      HRF_TRY(launch_asm_mac_distance(spec, channels, M, pixel_pitch, wavelengths, distances[d],
                                      aperture, false, false, buf, s));
    }
    {
      HRF_STAGE("asm_fft", s);
      HRF_TRY(fft_c2c(buf, M, channels, true, s));
    }
    {
      HRF_STAGE("asm_crop", s);
      HRF_TRY(launch_asm_crop(buf, channels, M, size, size,
                              static_cast<float>(1.0 / static_cast<double>(MM)),
                              static_cast<float2*>(out) + d * channels * SS, s));
    }
  }
  return HRF_OK;
}

int hrf_asm_multidistance_adjoint(const void* grad_out, int32_t num_distances, int32_t channels,
                                  int32_t height, int32_t width, int32_t size,
                                  const float* wavelengths, const float* distances,
                                  double pixel_pitch, float aperture, void* grad_field,
                                  void* ws, size_t ws_bytes, void* stream) {
  HRF_TRY(check_asm(1, channels, height, width, size));
  if (num_distances < 1 || !grad_out || !wavelengths || !distances || !grad_field) {
    set_error("asm multi-distance: null pointer or no distance");
    return HRF_ERR_INVALID;
  }
  HRF_TRY(check_ws(ws, ws_bytes, hrf_asm_multidistance_workspace_size(channels, size),
                   "asm multi-distance"));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int M = 2 * size;
  const int64_t MM = static_cast<int64_t>(M) * M;
  const int64_t SS = static_cast<int64_t>(size) * size;
  Carver cv(ws);
  float2* acc = cv.take<float2>(static_cast<size_t>(channels) * MM);
  float2* buf = cv.take<float2>(static_cast<size_t>(channels) * MM);
  if (fused_fft_supported(M)) {
    // X = acc holds the row spectra of 2 distances' gradients at a time
    // (C * size * M each); buf holds the (C, H, M) column-pass sum.
    return fused_md_adjoint(static_cast<const float2*>(grad_out), num_distances, channels,
                            height, width, size, pixel_pitch, wavelengths, distances, aperture,
                            static_cast<float2*>(grad_field), acc, buf, M / size, s);
  }
  // sum_d conj(T_d) FFT(pad g_d) in the spectral domain, one inverse FFT.
  for (int d = 0; d < num_distances; ++d) {
    {
      HRF_STAGE("asm_pad", s);
      HRF_TRY(launch_asm_pad(static_cast<const float2*>(grad_out) + d * channels * SS,
                             channels, size, size, buf, M, s));
    }
    {
      HRF_STAGE("asm_fft", s);
      HRF_TRY(fft_c2c(buf, M, channels, false, s));
    }
    {
      HRF_STAGE("asm_mac_adj", s);
      HRF_TRY(launch_asm_mac_distance(buf, channels, M, pixel_pitch, wavelengths, distances[d],
                                      aperture, true, d > 0, acc, s));
    }
  }
  {
    HRF_STAGE("asm_fft", s);
    HRF_TRY(fft_c2c(acc, M, channels, true, s));
  }
  {
    HRF_STAGE("asm_crop", s);
    HRF_TRY(launch_asm_crop(acc, channels, M, height, width,
                            static_cast<float>(1.0 / static_cast<double>(MM)),
                            static_cast<float2*>(grad_field), s));
  }
  return HRF_OK;
}

int hrf_asm_forward(const void* field, int32_t height, int32_t width, int32_t size,
                    float wavelength, double pixel_pitch, float distance, float aperture,
                    void* out, void* ws, size_t ws_bytes, void* stream) {
  return hrf_asm_multiplane_forward(field, 1, 1, height, width, size, &wavelength, &distance,
                                    pixel_pitch, aperture, out, ws, ws_bytes, stream);
}

int hrf_asm_adjoint(const void* grad_out, int32_t height, int32_t width, int32_t size,
                    float wavelength, double pixel_pitch, float distance, float aperture,
                    void* grad_field, void* ws, size_t ws_bytes, void* stream) {
  return hrf_asm_multiplane_adjoint(grad_out, 1, 1, height, width, size, &wavelength,
                                    &distance, pixel_pitch, aperture, grad_field, ws, ws_bytes,
                                    stream);
}

void hrf_release_caches(void) {
  hrf::fft_release_all();
  hrf::fused_fft_release_all();
}

}  // extern "C"
