/*
 * hrf_oracle.c — CPU restatement of the reference's complex wave rasterizer
 * and band-limited ASM spectral kernel.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker: it may be
 * built, loaded and called only by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg.  The product (the HIP library) never links
 * or calls it.
 *
 * It restates, literally and in the reference's evaluation order, the CUDA
 * code of complight/Complex_Valued_Holographic_Radiance_Fields:
 *   cuda_prop/cov3d_cuda/wave_rasterizer/forward.cu        (means2D, J, Sigma, cov2D)
 *   cuda_prop/cov3d_cuda/wave_rasterizer/forward_splat.cu  (preprocess, render)
 *   cuda_prop/cov3d_cuda/wave_rasterizer/auxiliary.h       (getRect)
 *   cuda_prop/cov3d_cuda/wave_rasterizer/rasterizer_splat.cu (keys, sort, ranges)
 *   cuda_prop/cov3d_cuda/wave_rasterizer/backward_splat.cu (render backward)
 *   cuda_prop/cov3d_cuda/wave_rasterizer/backward.cu       (geometry backward)
 *   cuda_prop/cuda/bandlimited_propagation_cuda.cu         (ASM spectral kernel)
 * Arithmetic model: every scalar expression is evaluated in source order with
 * IEEE single precision and no contraction (build with -ffp-contract=off);
 * the cuBLAS matmul chain (torch::matmul, forward.cu:265-268,
 * backward.cu:426-439) is a left-to-right fmaf dot product over k.  The
 * reference's __sincosf (fast intrinsic) is replaced by the accurate
 * sincosf; expf is libm's.  Backward gradients are accumulated in double
 * (the reference uses float atomics in an unspecified order).
 */
#define _GNU_SOURCE /* sincosf */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define TILE 16
#define PLANE_CUTOFF 1e-6f
#define MAX_ALPHA 0.99f

/* ----------------------------------------------------------- projection */

static float dot3(float a0, float b0, float a1, float b1, float a2, float b2) {
  return fmaf(a2, b2, fmaf(a1, b1, a0 * b0));
}
static float dot2(float a0, float b0, float a1, float b1) { return fmaf(a1, b1, a0 * b0); }

/* GLM mat3 product: Res[c][r] = A[0][r]*B[c][0] + A[1][r]*B[c][1] + A[2][r]*B[c][2]
 * (third_party/glm/glm/detail/type_mat3x3.inl:486-516). */
static void glm_mul(const float A[3][3], const float B[3][3], float R[3][3]) {
  for (int c = 0; c < 3; ++c)
    for (int r = 0; r < 3; ++r) R[c][r] = A[0][r] * B[c][0] + A[1][r] * B[c][1] + A[2][r] * B[c][2];
}

/* forward.cu:23-45, backward.cu:102-124: normalise q, GLM rotation (column
 * major constructor: R[c][r] = value 3c+r of the listed nine). */
static void rotation(const float* q, float R[3][3], float* rn, float* xn, float* yn, float* zn) {
  float r = q[0], x = q[1], y = q[2], z = q[3];
  const float norm = sqrtf(r * r + x * x + y * y + z * z);
  r /= norm;
  x /= norm;
  y /= norm;
  z /= norm;
  R[0][0] = 1.f - 2.f * (y * y + z * z);
  R[0][1] = 2.f * (x * y - r * z);
  R[0][2] = 2.f * (x * z + r * y);
  R[1][0] = 2.f * (x * y + r * z);
  R[1][1] = 1.f - 2.f * (x * x + z * z);
  R[1][2] = 2.f * (y * z - r * x);
  R[2][0] = 2.f * (x * z - r * y);
  R[2][1] = 2.f * (y * z + r * x);
  R[2][2] = 1.f - 2.f * (x * x + y * y);
  *rn = r;
  *xn = x;
  *yn = y;
  *zn = z;
}

static void diag3(const float* s, float S[3][3]) {
  memset(S, 0, sizeof(float) * 9);
  S[0][0] = s[0];
  S[1][1] = s[1];
  S[2][2] = s[2];
}

/* compute_cov3d_cuda_kernel (forward.cu:9-61): out[i*3+j] = Sigma[i][j]. */
void oracle_cov3d(const float* q, const float* s, float* out9) {
  float R[3][3], S[3][3], SR[3][3], SRt[3][3], Sg[3][3];
  float r, x, y, z;
  rotation(q, R, &r, &x, &y, &z);
  diag3(s, S);
  glm_mul(S, R, SR);
  for (int c = 0; c < 3; ++c)
    for (int rr = 0; rr < 3; ++rr) SRt[c][rr] = SR[rr][c];
  glm_mul(SRt, SR, Sg);
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) out9[i * 3 + j] = Sg[i][j];
}

/* compute_jacobian_kernel (forward.cu:64-122). Returns 0 when clipped. */
static int jacobian(float tx, float ty, float tz, float fx, float fy, float lim_x, float lim_y,
                    float near_p, float far_p, float J[2][3]) {
  if (tz <= near_p || tz >= far_p) {
    memset(J, 0, sizeof(float) * 6);
    return 0;
  }
  const float tz2 = tz * tz;
  const float tx_tz = tx / tz;
  const float ty_tz = ty / tz;
  const float ctx = fminf(fmaxf(tx_tz, -lim_x), lim_x);
  const float cty = fminf(fmaxf(ty_tz, -lim_y), lim_y);
  const float cx = ctx * tz;
  const float cy = cty * tz;
  J[0][0] = fx / tz;
  J[0][1] = 0.0f;
  J[0][2] = -(fx * cx) / tz2;
  J[1][0] = 0.0f;
  J[1][1] = fy / tz;
  J[1][2] = -(fy * cy) / tz2;
  return 1;
}

static void lims(int W, int H, float fx, float fy, float* lim_x, float* lim_y) {
  /* half_tan_fov = 0.5f * width / fx (forward.cu:199-200); lim = 1.3f * it. */
  const float htx = 0.5f * (float)W / fx;
  const float hty = 0.5f * (float)H / fy;
  *lim_x = 1.3f * htx;
  *lim_y = 1.3f * hty;
}

/* compute_cov2d_forward (forward.cu:221-294). */
static void cov2d_chain(const float J[2][3], const float Wm[3][3], const float sig[3][3],
                        float JW[2][3], float cov[2][2]) {
  float M1[2][3], M2[2][3];
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 3; ++j) JW[i][j] = dot3(J[i][0], Wm[0][j], J[i][1], Wm[1][j], J[i][2], Wm[2][j]);
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 3; ++j)
      M1[i][j] = dot3(JW[i][0], sig[0][j], JW[i][1], sig[1][j], JW[i][2], sig[2][j]);
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 3; ++j) M2[i][j] = dot3(M1[i][0], Wm[j][0], M1[i][1], Wm[j][1], M1[i][2], Wm[j][2]);
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 2; ++j) cov[i][j] = dot3(M2[i][0], J[j][0], M2[i][1], J[j][1], M2[i][2], J[j][2]);
  cov[0][0] += 0.3f;
  cov[1][1] += 0.3f;
}

/* Projection of all Gaussians: means2D (N,2), J (N,6), Sigma (N,9), JW (N,6),
 * cov2D (N,4).  Any output pointer may be NULL. */
void oracle_project(int64_t n, const float* cam, const float* quats, const float* scales,
                    const float* view, float fx, float fy, float px, float py, int W, int H,
                    float near_p, float far_p, float* means2d, float* Jout, float* sigout,
                    float* JWout, float* cov2d) {
  float lim_x, lim_y;
  lims(W, H, fx, fy, &lim_x, &lim_y);
  float Wm[3][3];
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) Wm[i][j] = view[i * 3 + j];
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < n; ++g) {
    const float tx = cam[g * 3 + 0], ty = cam[g * 3 + 1], tz = cam[g * 3 + 2];
    if (means2d) {
      /* compute_means2d_kernel (forward.cu:297-330) */
      if (tz <= near_p || tz >= far_p) {
        means2d[g * 2 + 0] = 1e6f;
        means2d[g * 2 + 1] = 1e6f;
      } else {
        const float inv_z = 1.0f / tz;
        const float px_div = -tx * inv_z;
        const float py_div = -ty * inv_z;
        means2d[g * 2 + 0] = fx * px_div + px;
        means2d[g * 2 + 1] = fy * py_div + py;
      }
    }
    float J[2][3], sig9[9], sig[3][3], JW[2][3], cv[2][2];
    jacobian(tx, ty, tz, fx, fy, lim_x, lim_y, near_p, far_p, J);
    oracle_cov3d(quats + g * 4, scales + g * 3, sig9);
    for (int i = 0; i < 3; ++i)
      for (int j = 0; j < 3; ++j) sig[i][j] = sig9[i * 3 + j];
    cov2d_chain(J, Wm, sig, JW, cv);
    if (Jout) memcpy(Jout + g * 6, J, sizeof(float) * 6);
    if (sigout) memcpy(sigout + g * 9, sig9, sizeof(float) * 9);
    if (JWout) memcpy(JWout + g * 6, JW, sizeof(float) * 6);
    if (cov2d) {
      cov2d[g * 4 + 0] = cv[0][0];
      cov2d[g * 4 + 1] = cv[0][1];
      cov2d[g * 4 + 2] = cv[1][0];
      cov2d[g * 4 + 3] = cv[1][1];
    }
  }
}

/* ------------------------------------------------------------- binning */

static uint32_t to_u32_sat(float f) {
  /* (uint32_t) of a float as the reference's GPU cast behaves: truncation,
   * negatives/NaN -> 0, overflow -> max (C leaves these undefined). */
  if (!(f > 0.0f)) return 0u;
  if (f >= 4294967296.0f) return 0xFFFFFFFFu;
  return (uint32_t)f;
}

/* preprocessGaussiansKernel (forward_splat.cu:17-98) + getRect
 * (auxiliary.h:119-137).  rect = (minx, miny, maxx, maxy) per Gaussian.
 * A non-positive or NaN radius (degenerate covariance; undefined in the
 * reference) or a NaN 2-D mean culls the Gaussian. */
void oracle_preprocess(int64_t n, const float* means2d, const float* cov2d, const float* z,
                       int W, int H, float near_p, float far_p, int32_t* radii,
                       uint32_t* tiles, uint32_t* rect) {
  const uint32_t gx = (uint32_t)((W + TILE - 1) / TILE), gy = (uint32_t)((H + TILE - 1) / TILE);
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < n; ++g) {
    radii[g] = 0;
    tiles[g] = 0;
    if (rect) rect[g * 4 + 0] = rect[g * 4 + 1] = rect[g * 4 + 2] = rect[g * 4 + 3] = 0;
    const float zz = z[g];
    if (zz <= near_p || zz >= far_p) continue;
    float cx = cov2d[g * 4 + 0], cy = cov2d[g * 4 + 1], cz = cov2d[g * 4 + 2], cw = cov2d[g * 4 + 3];
    float det_cov = cx * cw - cy * cz;
    if (fabsf(det_cov) < 1e-10f) continue;
    cx += 0.3f;
    cw += 0.3f;
    det_cov = cx * cw - cy * cz;
    const float det = det_cov;
    if (fabsf(det) < 1e-8f) continue;
    const float mid = 0.5f * (cx + cw);
    const float disc = fmaxf(0.1f, mid * mid - det);
    const float lambda1 = mid + sqrtf(disc);
    const float lambda2 = mid - sqrtf(disc);
    const float radius_f = ceilf(3.0f * sqrtf(fmaxf(lambda1, lambda2)));
    if (!(radius_f > 0.0f)) continue;
    /* A NaN 2-D mean (NaN camera-space x or y: the Jacobian's clamp keeps
     * the covariance finite) would fall in tile 0 and composite with alpha
     * fminf(0.99, NaN) = 0.99; it is culled like a NaN radius. */
    if (isnan(means2d[g * 2 + 0]) || isnan(means2d[g * 2 + 1])) continue;
    const int rad_i = radius_f < 2147483520.0f ? (int)radius_f : 2147483520;
    radii[g] = rad_i;
    const int radius = rad_i > 1 ? rad_i : 1;
    const float rf = (float)radius;
    const float mx = means2d[g * 2 + 0], my = means2d[g * 2 + 1];
    uint32_t minx = to_u32_sat((mx - rf) / 16.0f);
    uint32_t miny = to_u32_sat((my - rf) / 16.0f);
    minx = minx < gx - 1 ? minx : gx - 1;
    miny = miny < gy - 1 ? miny : gy - 1;
    uint32_t maxx = to_u32_sat((mx + rf + 16.0f - 1.0f) / 16.0f);
    uint32_t maxy = to_u32_sat((my + rf + 16.0f - 1.0f) / 16.0f);
    maxx = maxx > 1u ? maxx : 1u;
    maxy = maxy > 1u ? maxy : 1u;
    maxx = maxx < gx ? maxx : gx;
    maxy = maxy < gy ? maxy : gy;
    if (maxx <= minx) maxx = (minx + 1 < gx) ? minx + 1 : gx;
    if (maxy <= miny) maxy = (miny + 1 < gy) ? miny + 1 : gy;
    tiles[g] = (maxy - miny) * (maxx - minx);
    if (rect) {
      rect[g * 4 + 0] = minx;
      rect[g * 4 + 1] = miny;
      rect[g * 4 + 2] = maxx;
      rect[g * 4 + 3] = maxy;
    }
  }
}

typedef struct {
  uint64_t key;
  uint32_t val;
} KV;

static int kv_cmp(const void* a, const void* b) {
  const KV* x = (const KV*)a;
  const KV* y = (const KV*)b;
  if (x->key != y->key) return x->key < y->key ? -1 : 1;
  /* stable: the unsorted array is in Gaussian-index order, so ties keep
   * index order (cub::DeviceRadixSort is stable). */
  if (x->val != y->val) return x->val < y->val ? -1 : 1;
  return 0;
}

/* Pair count for a scene (sum of tiles), so the caller can size buffers. */
int64_t oracle_count_pairs(int64_t n, const uint32_t* tiles) {
  int64_t k = 0;
  for (int64_t g = 0; g < n; ++g) k += tiles[g];
  return k;
}

/* duplicateWithKeysKernel + SortPairs + identifyTileRangesKernel
 * (rasterizer_splat.cu:114-201,457-495).  point_list (K) int32, ranges
 * (T,2) int32 (empty tiles (0,0)). */
void oracle_bin(int64_t n, const float* z, const uint32_t* tiles, const uint32_t* rect, int W,
                int H, int64_t k, int32_t* point_list, int32_t* ranges) {
  const uint32_t gx = (uint32_t)((W + TILE - 1) / TILE), gy = (uint32_t)((H + TILE - 1) / TILE);
  const int64_t ntiles = (int64_t)gx * gy;
  memset(ranges, 0, sizeof(int32_t) * 2 * ntiles);
  if (k == 0) return;
  KV* kv = (KV*)malloc(sizeof(KV) * (size_t)k);
  int64_t off = 0;
  for (int64_t g = 0; g < n; ++g) {
    if (tiles[g] == 0) continue;
    uint32_t bits;
    memcpy(&bits, &z[g], 4);
    bits = (bits & 0x80000000u) ? (bits & 0x7FFFFFFFu) : (bits | 0x80000000u);
    for (uint32_t y = rect[g * 4 + 1]; y < rect[g * 4 + 3]; ++y)
      for (uint32_t x = rect[g * 4 + 0]; x < rect[g * 4 + 2]; ++x) {
        kv[off].key = ((uint64_t)(y * gx + x) << 32) | bits;
        kv[off].val = (uint32_t)g;
        ++off;
      }
  }
  qsort(kv, (size_t)k, sizeof(KV), kv_cmp);
  for (int64_t i = 0; i < k; ++i) {
    point_list[i] = (int32_t)kv[i].val;
    const uint32_t t = (uint32_t)(kv[i].key >> 32);
    if (i == 0 || (uint32_t)(kv[i - 1].key >> 32) != t) ranges[2 * t] = (int32_t)i;
    if (i == k - 1 || (uint32_t)(kv[i + 1].key >> 32) != t) ranges[2 * t + 1] = (int32_t)(i + 1);
  }
  free(kv);
}

/* ------------------------------------------------------- forward render */

/* renderTileKernel (forward_splat.cu:101-289), defined semantics: every
 * pixel of a partial edge tile sees the full batch (the reference leaves
 * LDS slots of out-of-image threads unloaded).  field is (P,C,H,W) complex
 * interleaved (re, im); final_T and n_contrib (P,H,W).  tile_mask (one byte
 * per tile, may be NULL = every tile): pixels of tiles whose byte is 0 are
 * skipped and their outputs left as they are. */
void oracle_render_forward(int W, int H, int P, int C, const int32_t* ranges,
                           const int32_t* point_list, const float* means2d, const float* cov2d,
                           const float* z, const float* colours, const float* phase,
                           const float* opac, const float* pprobs, float near_p, float far_p,
                           float* field, float* final_T, int32_t* n_contrib,
                           const uint8_t* tile_mask) {
  const int gx = (W + TILE - 1) / TILE;
  const int64_t HW = (int64_t)W * H;
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t pix = 0; pix < HW; ++pix) {
    const int py = (int)(pix / W), px = (int)(pix % W);
    const int tile = (py / TILE) * gx + (px / TILE);
    if (tile_mask && !tile_mask[tile]) continue;
    const int r0 = ranges[2 * tile], r1 = ranges[2 * tile + 1];
    const float pxf = (float)px, pyf = (float)py;
    for (int p = 0; p < P; ++p) {
      float T = 1.0f;
      uint32_t position = 0, last_position = 0;
      float ar[3] = {0.f, 0.f, 0.f}, ai[3] = {0.f, 0.f, 0.f};
      for (int k = r0; k < r1; ++k) {
        position++;
        const int g = point_list[k];
        const float zz = z[g];
        if (zz <= near_p || zz >= far_p) continue;
        const float w = pprobs[(int64_t)g * P + p];
        if (w < PLANE_CUTOFF) continue;
        const float dx = means2d[g * 2 + 0] - pxf, dy = means2d[g * 2 + 1] - pyf;
        const float cx = cov2d[g * 4 + 0], cy = cov2d[g * 4 + 1], cz = cov2d[g * 4 + 2],
                    cw = cov2d[g * 4 + 3];
        const float det = cx * cw - cy * cz;
        const float det_inv = 1.0f / det;
        const float inv00 = cw * det_inv;
        const float inv01 = -cy * det_inv;
        const float inv10 = -cz * det_inv;
        const float inv11 = cx * det_inv;
        const float power = -0.5f * (dx * (inv00 * dx + inv10 * dy) + dy * (inv01 * dx + inv11 * dy));
        if (power > 0.0f) continue;
        const float o = opac[g];
        const float gexp = expf(power);
        const float alpha = fminf(MAX_ALPHA, o * gexp * w);
        const float test_T = T * (1.0f - alpha);
        const int done = test_T < 0.0001f;
        for (int c = 0; c < C; ++c) {
          const float color = colours[(int64_t)g * C + c];
          const float ph = phase[(int64_t)g * C + c];
          const float scale = color * alpha * T;
          float sv, cv;
          sincosf(ph, &sv, &cv);
          ar[c] += scale * cv;
          ai[c] += scale * sv;
        }
        T = test_T;
        last_position = position;
        if (done) break;
      }
      for (int c = 0; c < C; ++c) {
        const int64_t idx = ((int64_t)p * C + c) * HW + pix;
        field[2 * idx] = ar[c];
        field[2 * idx + 1] = ai[c];
      }
      final_T[(int64_t)p * HW + pix] = T;
      n_contrib[(int64_t)p * HW + pix] = (int32_t)last_position;
    }
  }
}

/* ------------------------------------------------------ backward render */

/* renderBackwardTileKernel (backward_splat.cu:78-307).  grad_field (P,C,H,W)
 * complex interleaved.  Outputs (double accumulators, zeroed here):
 * g_means2d (N,2), g_cov2d (N,4), g_col (N,C), g_phase (N,C), g_opac (N),
 * g_plane (N,P).  tile_mask as in oracle_render_forward: only the pixels of
 * the selected tiles contribute.
 *
 * The (tile, plane) pairs run in parallel, each summing its pixels' terms
 * into doubles indexed by tile-list position (pixels in row-major order
 * within the tile); those partial sums are then added into the
 * per-Gaussian accumulators in (tile, plane, position) order, so the result
 * does not depend on the thread count.  The per-pixel float arithmetic is
 * the reference's, in its order. */
enum { BW_MX, BW_MY, BW_CXX, BW_CXY, BW_CYY, BW_OPAC, BW_PLANE, BW_COL };

static void render_backward_tile_plane(int W, int H, int P, int C, int tile, int p, int r0,
                                       int r1, const int32_t* point_list,
                                       const float* means2d, const float* cov2d,
                                       const float* colours, const float* phase,
                                       const float* opac, const float* pprobs,
                                       const float* final_T, const int32_t* n_contrib,
                                       const float* grad_field, double* acc, int nv) {
  const int gx = (W + TILE - 1) / TILE;
  const int64_t HW = (int64_t)W * H;
  const float ddelx_dx = 0.5f * (float)W;
  const float ddely_dy = 0.5f * (float)H;
  const int tx = tile % gx, ty = tile / gx;
  for (int py = ty * TILE; py < ty * TILE + TILE && py < H; ++py)
    for (int px = tx * TILE; px < tx * TILE + TILE && px < W; ++px) {
      const int64_t pix = (int64_t)py * W + px;
      const float pxf = (float)px, pyf = (float)py;
      float gre[3], gim[3];
      for (int c = 0; c < C; ++c) {
        const int64_t idx = ((int64_t)p * C + c) * HW + pix;
        gre[c] = grad_field[2 * idx];
        gim[c] = grad_field[2 * idx + 1];
      }
      float T = final_T[(int64_t)p * HW + pix];
      const int last = n_contrib[(int64_t)p * HW + pix];
      float accr[3] = {0, 0, 0}, acci[3] = {0, 0, 0}, lastr[3] = {0, 0, 0}, lasti[3] = {0, 0, 0};
      float last_alpha = 0.0f;
      for (int k = r1 - 1; k >= r0; --k) {
        const int contributor = k - r0; /* 0-based position in the tile list */
        if (contributor >= last) continue;
        const int g = point_list[k];
        double* a = acc + (int64_t)contributor * nv;
        const float w = pprobs[(int64_t)g * P + p];
        if (w < PLANE_CUTOFF) continue;
        const float dx = means2d[g * 2 + 0] - pxf, dy = means2d[g * 2 + 1] - pyf;
        const float cx = cov2d[g * 4 + 0], cy = cov2d[g * 4 + 1], cz = cov2d[g * 4 + 2],
                    cw = cov2d[g * 4 + 3];
        const float det = cx * cw - cy * cz;
        if (det == 0.0f) continue;
        const float det_inv = 1.0f / det;
        const float conic_x = cw * det_inv;
        const float conic_y = -cy * det_inv;
        const float conic_z = cx * det_inv;
        const float power = -0.5f * (conic_x * dx * dx + conic_z * dy * dy) - conic_y * dx * dy;
        if (power > 0.0f) continue;
        const float o = opac[g];
        const float G = expf(power);
        const float alpha = fminf(0.99f, o * G * w);
        if (alpha < 1.0f / 255.0f) continue;
        T = T / (1.0f - alpha);
        const float dchannel_dcolor = alpha * T;
        float dL_dalpha = 0.0f;
        for (int c = 0; c < C; ++c) {
          const float color = colours[(int64_t)g * C + c];
          const float ph = phase[(int64_t)g * C + c];
          float sn, cs;
          sincosf(ph, &sn, &cs);
          const float color_real = color * cs;
          const float color_imag = color * sn;
          accr[c] = last_alpha * lastr[c] + (1.0f - last_alpha) * accr[c];
          acci[c] = last_alpha * lasti[c] + (1.0f - last_alpha) * acci[c];
          lastr[c] = color_real;
          lasti[c] = color_imag;
          dL_dalpha += (color_real - accr[c]) * gre[c];
          dL_dalpha += (color_imag - acci[c]) * gim[c];
          const float dL_dcolor = dchannel_dcolor * (cs * gre[c] + sn * gim[c]);
          a[BW_COL + c] += dL_dcolor;
          const float dL_dphase = dchannel_dcolor * color * (-sn * gre[c] + cs * gim[c]);
          a[BW_COL + C + c] += dL_dphase;
        }
        dL_dalpha *= T;
        last_alpha = alpha;
        const float dL_dG = o * w * dL_dalpha;
        const float gdx = G * dx;
        const float gdy = G * dy;
        const float dG_ddelx = -gdx * conic_x - gdy * conic_y;
        const float dG_ddely = -gdy * conic_z - gdx * conic_y;
        a[BW_MX] += dL_dG * dG_ddelx * ddelx_dx;
        a[BW_MY] += dL_dG * dG_ddely * ddely_dy;
        const float dL_dconic_x = -0.5f * gdx * dx * dL_dG;
        const float dL_dconic_y = -0.5f * gdx * dy * dL_dG;
        const float dL_dconic_z = -0.5f * gdy * dy * dL_dG;
        const float dL_dcov_xx = dL_dconic_x * (cw * det_inv * det_inv) * cw +
                                 dL_dconic_z * (-cy * det_inv * det_inv) * (-cy);
        const float dL_dcov_xy = dL_dconic_x * (cw * det_inv * det_inv) * (-cy) +
                                 dL_dconic_y * (-det_inv) +
                                 dL_dconic_z * (-cy * det_inv * det_inv) * cx;
        const float dL_dcov_yy = dL_dconic_x * (-cy * det_inv * det_inv) * (-cy) +
                                 dL_dconic_z * (cx * det_inv * det_inv) * cx;
        a[BW_CXX] += dL_dcov_xx;
        a[BW_CXY] += dL_dcov_xy; /* the reference adds it to both off-diagonals */
        a[BW_CYY] += dL_dcov_yy;
        a[BW_OPAC] += G * w * dL_dalpha;
        a[BW_PLANE] += o * G * dL_dalpha;
      }
    }
}

void oracle_render_backward(int64_t n, int W, int H, int P, int C, const int32_t* ranges,
                            const int32_t* point_list, const float* means2d,
                            const float* cov2d, const float* colours, const float* phase,
                            const float* opac, const float* pprobs, const float* final_T,
                            const int32_t* n_contrib, const float* grad_field,
                            double* g_means2d, double* g_cov2d, double* g_col, double* g_phase,
                            double* g_opac, double* g_plane, const uint8_t* tile_mask) {
  const int gx = (W + TILE - 1) / TILE, gy = (H + TILE - 1) / TILE;
  const int64_t njobs = (int64_t)gx * gy * P;
  const int nv = BW_COL + 2 * C;
  memset(g_means2d, 0, sizeof(double) * 2 * n);
  memset(g_cov2d, 0, sizeof(double) * 4 * n);
  memset(g_col, 0, sizeof(double) * C * n);
  memset(g_phase, 0, sizeof(double) * C * n);
  memset(g_opac, 0, sizeof(double) * n);
  memset(g_plane, 0, sizeof(double) * P * n);
  double** part = (double**)calloc((size_t)(njobs > 0 ? njobs : 1), sizeof(double*));
  if (!part) abort();
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t job = 0; job < njobs; ++job) {
    const int tile = (int)(job / P), p = (int)(job % P);
    if (tile_mask && !tile_mask[tile]) continue;
    const int r0 = ranges[2 * tile], r1 = ranges[2 * tile + 1];
    if (r1 <= r0) continue;
    double* acc = (double*)calloc((size_t)(r1 - r0) * nv, sizeof(double));
    if (!acc) abort();
    render_backward_tile_plane(W, H, P, C, tile, p, r0, r1, point_list, means2d, cov2d, colours,
                               phase, opac, pprobs, final_T, n_contrib, grad_field, acc, nv);
    part[job] = acc;
  }
  for (int64_t job = 0; job < njobs; ++job) {
    double* acc = part[job];
    if (!acc) continue;
    const int tile = (int)(job / P), p = (int)(job % P);
    const int r0 = ranges[2 * tile], r1 = ranges[2 * tile + 1];
    for (int k = r0; k < r1; ++k) {
      const double* a = acc + (int64_t)(k - r0) * nv;
      const int64_t g = point_list[k];
      g_means2d[g * 2 + 0] += a[BW_MX];
      g_means2d[g * 2 + 1] += a[BW_MY];
      g_cov2d[g * 4 + 0] += a[BW_CXX];
      g_cov2d[g * 4 + 1] += a[BW_CXY];
      g_cov2d[g * 4 + 2] += a[BW_CXY];
      g_cov2d[g * 4 + 3] += a[BW_CYY];
      for (int c = 0; c < C; ++c) {
        g_col[g * C + c] += a[BW_COL + c];
        g_phase[g * C + c] += a[BW_COL + C + c];
      }
      g_opac[g] += a[BW_OPAC];
      g_plane[g * P + p] += a[BW_PLANE];
    }
    free(acc);
  }
  free(part);
}

/* ----------------------------------------------------- geometry backward */

/* BACKWARD_SPLAT::preprocess (backward_splat.cu:364-417) with
 * compute_means2d_backward (backward.cu:453-497), compute_cov2d_backward
 * (:363-450), compute_jacobian_backward (:201-272) and
 * compute_cov3d_backward (:21-198).  Inputs are the float grads of
 * means2D (N,2) and cov2D (N,4); outputs grad_cam (N,3), grad_quat (N,4),
 * grad_scale (N,3).  Also exposes dL_dSigma (N,9) and dL_dJ (N,6) if
 * non-NULL (for the unit tests of each chain link). */
/* means2D backward (backward.cu:453-497); zero when clipped. */
static void means2d_bwd(float tx, float ty, float tz, float fx, float fy, float near_p,
                        float far_p, float gx_, float gy_, float g[3]) {
  g[0] = g[1] = g[2] = 0.f;
  if (tz <= near_p || tz >= far_p) return;
  const float z2 = tz * tz;
  g[0] = -fx * gx_ / tz;
  g[1] = -fy * gy_ / tz;
  g[2] = (fx * tx * gx_ / z2) + (fy * ty * gy_ / z2);
}

/* cov2D chain backward (backward.cu:426-439): dL_dC = G2 J, dL_dB = dL_dC W,
 * dL_dSigma = JW^T (G2 JW), dL_dA = dL_dB Sigma^T, dL_dJ = dL_dA W^T. */
static void cov2d_chain_bwd(const float G2[2][2], const float J[2][3], const float Wm[3][3],
                            const float sig[3][3], const float JW[2][3], float dSig[3][3],
                            float dJ[2][3]) {
  float dC[2][3], dB[2][3], X[2][3], dA[2][3];
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 3; ++j) dC[i][j] = dot2(G2[i][0], J[0][j], G2[i][1], J[1][j]);
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 3; ++j) dB[i][j] = dot3(dC[i][0], Wm[0][j], dC[i][1], Wm[1][j], dC[i][2], Wm[2][j]);
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 3; ++j) X[i][j] = dot2(G2[i][0], JW[0][j], G2[i][1], JW[1][j]);
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) dSig[i][j] = dot2(JW[0][i], X[0][j], JW[1][i], X[1][j]);
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 3; ++j) dA[i][j] = dot3(dB[i][0], sig[j][0], dB[i][1], sig[j][1], dB[i][2], sig[j][2]);
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 3; ++j) dJ[i][j] = dot3(dA[i][0], Wm[j][0], dA[i][1], Wm[j][1], dA[i][2], Wm[j][2]);
}

/* compute_jacobian_backward_kernel (backward.cu:201-272): clamp mask, but
 * the unclamped tx/ty in dJ02/dtz, dJ12/dtz; zero when clipped. */
static void jacobian_bwd(float tx, float ty, float tz, float fx, float fy, float lim_x,
                         float lim_y, float near_p, float far_p, const float dJ[2][3], float g[3]) {
  g[0] = g[1] = g[2] = 0.f;
  if (tz <= near_p || tz >= far_p) return;
  const float tz2 = tz * tz;
  const float tz3 = tz2 * tz;
  const float tx_tz = tx / tz;
  const float ty_tz = ty / tz;
  const float xm = (tx_tz < -lim_x || tx_tz > lim_x) ? 0.0f : 1.0f;
  const float ym = (ty_tz < -lim_y || ty_tz > lim_y) ? 0.0f : 1.0f;
  const float dJ00_dtz = -fx / tz2;
  const float dJ02_dtx = xm * (-fx / tz2);
  const float dJ02_dtz = xm * (2.0f * fx * tx / tz3);
  const float dJ11_dtz = -fy / tz2;
  const float dJ12_dty = ym * (-fy / tz2);
  const float dJ12_dtz = ym * (2.0f * fy * ty / tz3);
  g[0] = dJ[0][2] * dJ02_dtx;
  g[1] = dJ[1][2] * dJ12_dty;
  g[2] = dJ[0][0] * dJ00_dtz + dJ[0][2] * dJ02_dtz + dJ[1][1] * dJ11_dtz + dJ[1][2] * dJ12_dtz;
}

/* compute_cov3d_backward_cuda_kernel (backward.cu:76-198): Gm[i][j] =
 * grad[i*3+j] read as GLM column i, row j; grad_s = (2 R^T G R)[k][k] s[k];
 * grad_q = elementwise sums over S * dR/dq (backward.cu:31-73,161-187). */
static void cov3d_bwd(const float Gm[3][3], const float* q, const float* s, float gq[4],
                      float gs[3]) {
  float R[3][3], S[3][3];
  float r, x, y, z;
  rotation(q, R, &r, &x, &y, &z);
  diag3(s, S);
  const float dRr[3][3] = {{0.f, -2.f * z, 2.f * y}, {2.f * z, 0.f, -2.f * x}, {-2.f * y, 2.f * x, 0.f}};
  const float dRx[3][3] = {{0.f, 2.f * y, 2.f * z}, {2.f * y, -4.f * x, -2.f * r}, {2.f * z, 2.f * r, -4.f * x}};
  const float dRy[3][3] = {{-4.f * y, 2.f * x, 2.f * r}, {2.f * x, 0.f, 2.f * z}, {-2.f * r, 2.f * z, -4.f * y}};
  const float dRz[3][3] = {{-4.f * z, -2.f * r, 2.f * x}, {2.f * r, -4.f * z, 2.f * y}, {2.f * x, 2.f * y, 0.f}};
  float Rt2[3][3], T1[3][3], temp[3][3];
  for (int c = 0; c < 3; ++c)
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
  for (int i = 0; i < 3; ++i)
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

/* Fused geometry backward as the rasterizer backward uses it
 * (backward_splat.cu:364-417): means2D + cov2D chain + Jacobian + Sigma. */
void oracle_geom_backward(int64_t n, const float* cam, const float* quats, const float* scales,
                          const float* view, float fx, float fy, int W, int H, float near_p,
                          float far_p, const float* g_means2d, const float* g_cov2d,
                          float* g_cam, float* g_quat, float* g_scale, float* dsig_out,
                          float* dJ_out) {
  float lim_x, lim_y;
  lims(W, H, fx, fy, &lim_x, &lim_y);
  float Wm[3][3];
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) Wm[i][j] = view[i * 3 + j];
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < n; ++g) {
    const float tx = cam[g * 3 + 0], ty = cam[g * 3 + 1], tz = cam[g * 3 + 2];
    float J[2][3], sig9[9], sig[3][3], JW[2][3], cv[2][2];
    jacobian(tx, ty, tz, fx, fy, lim_x, lim_y, near_p, far_p, J);
    oracle_cov3d(quats + g * 4, scales + g * 3, sig9);
    for (int i = 0; i < 3; ++i)
      for (int j = 0; j < 3; ++j) sig[i][j] = sig9[i * 3 + j];
    cov2d_chain(J, Wm, sig, JW, cv);
    float gm[3], gj[3], dSig[3][3], dJ[2][3];
    means2d_bwd(tx, ty, tz, fx, fy, near_p, far_p, g_means2d[g * 2 + 0], g_means2d[g * 2 + 1], gm);
    const float G2[2][2] = {{g_cov2d[g * 4 + 0], g_cov2d[g * 4 + 1]},
                            {g_cov2d[g * 4 + 2], g_cov2d[g * 4 + 3]}};
    cov2d_chain_bwd(G2, J, Wm, sig, JW, dSig, dJ);
    if (dsig_out) memcpy(dsig_out + g * 9, dSig, sizeof(float) * 9);
    if (dJ_out) memcpy(dJ_out + g * 6, dJ, sizeof(float) * 6);
    jacobian_bwd(tx, ty, tz, fx, fy, lim_x, lim_y, near_p, far_p, dJ, gj);
    g_cam[g * 3 + 0] = gm[0] + gj[0];
    g_cam[g * 3 + 1] = gm[1] + gj[1];
    g_cam[g * 3 + 2] = gm[2] + gj[2];
    cov3d_bwd(dSig, quats + g * 4, scales + g * 3, g_quat + g * 4, g_scale + g * 3);
  }
}

/* ----------------------------------------- standalone geometry operators */

/* compute_cov3d_backward (backward.cu:274-320). */
void oracle_cov3d_backward(int64_t n, const float* grad9, const float* quats, const float* scales,
                           float* g_quat, float* g_scale) {
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < n; ++g) {
    float Gm[3][3];
    for (int i = 0; i < 3; ++i)
      for (int j = 0; j < 3; ++j) Gm[i][j] = grad9[g * 9 + i * 3 + j];
    cov3d_bwd(Gm, quats + g * 4, scales + g * 3, g_quat + g * 4, g_scale + g * 3);
  }
}

/* compute_jacobian_backward (backward.cu:322-361). */
void oracle_jacobian_backward(int64_t n, const float* grad6, const float* cam, float fx, float fy,
                              int W, int H, float near_p, float far_p, float* g_cam) {
  float lim_x, lim_y;
  lims(W, H, fx, fy, &lim_x, &lim_y);
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < n; ++g) {
    float dJ[2][3];
    for (int i = 0; i < 2; ++i)
      for (int j = 0; j < 3; ++j) dJ[i][j] = grad6[g * 6 + i * 3 + j];
    jacobian_bwd(cam[g * 3 + 0], cam[g * 3 + 1], cam[g * 3 + 2], fx, fy, lim_x, lim_y, near_p,
                 far_p, dJ, g_cam + g * 3);
  }
}

/* compute_cov2d_backward (backward.cu:363-450) on the saved J, Sigma, W, JW
 * as given; grad_cam from the Jacobian chain only. */
void oracle_cov2d_backward(int64_t n, const float* grad4, const float* cam, const float* quats,
                           const float* scales, const float* J6, const float* sig9,
                           const float* W9, const float* JW6, float fx, float fy, int W, int H,
                           float near_p, float far_p, float* g_cam, float* g_quat,
                           float* g_scale) {
  float lim_x, lim_y;
  lims(W, H, fx, fy, &lim_x, &lim_y);
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < n; ++g) {
    float J[2][3], sig[3][3], Wm[3][3], JW[2][3], dSig[3][3], dJ[2][3];
    for (int i = 0; i < 2; ++i)
      for (int j = 0; j < 3; ++j) {
        J[i][j] = J6[g * 6 + i * 3 + j];
        JW[i][j] = JW6[g * 6 + i * 3 + j];
      }
    for (int i = 0; i < 3; ++i)
      for (int j = 0; j < 3; ++j) {
        sig[i][j] = sig9[g * 9 + i * 3 + j];
        Wm[i][j] = W9[g * 9 + i * 3 + j];
      }
    const float G2[2][2] = {{grad4[g * 4 + 0], grad4[g * 4 + 1]}, {grad4[g * 4 + 2], grad4[g * 4 + 3]}};
    cov2d_chain_bwd(G2, J, Wm, sig, JW, dSig, dJ);
    jacobian_bwd(cam[g * 3 + 0], cam[g * 3 + 1], cam[g * 3 + 2], fx, fy, lim_x, lim_y, near_p,
                 far_p, dJ, g_cam + g * 3);
    cov3d_bwd(dSig, quats + g * 4, scales + g * 3, g_quat + g * 4, g_scale + g * 3);
  }
}

/* compute_means2d_backward (backward.cu:545-585). */
void oracle_means2d_backward(int64_t n, const float* grad2, const float* cam, float fx, float fy,
                             float near_p, float far_p, float* g_cam) {
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < n; ++g)
    means2d_bwd(cam[g * 3 + 0], cam[g * 3 + 1], cam[g * 3 + 2], fx, fy, near_p, far_p,
                grad2[g * 2 + 0], grad2[g * 2 + 1], g_cam + g * 3);
}

/* invert_cov2d_kernel (forward.cu:333-356). */
void oracle_invert_cov2d(int64_t n, const float* cov4, float* out4) {
  for (int64_t g = 0; g < n; ++g) {
    const float a = cov4[g * 4 + 0], b = cov4[g * 4 + 1], c = cov4[g * 4 + 2], d = cov4[g * 4 + 3];
    const float det = a * d - b * c;
    const float inv_det = 1.0f / det;
    out4[g * 4 + 0] = d * inv_det;
    out4[g * 4 + 1] = -b * inv_det;
    out4[g * 4 + 2] = -c * inv_det;
    out4[g * 4 + 3] = a * inv_det;
  }
}

/* invert_cov2d_backward_kernel (backward.cu:500-543): -(A^-1 (G A^-1)). */
void oracle_invert_cov2d_backward(int64_t n, const float* g4, const float* cov4, float* out4) {
  for (int64_t g = 0; g < n; ++g) {
    const float a = cov4[g * 4 + 0], b = cov4[g * 4 + 1], c = cov4[g * 4 + 2], d = cov4[g * 4 + 3];
    const float det = a * d - b * c;
    const float inv_det = 1.0f / det;
    const float ia = d * inv_det, ib = -b * inv_det, ic = -c * inv_det, id = a * inv_det;
    const float ga = g4[g * 4 + 0], gb = g4[g * 4 + 1], gc = g4[g * 4 + 2], gd = g4[g * 4 + 3];
    const float ta = ga * ia + gb * ic;
    const float tb = ga * ib + gb * id;
    const float tc = gc * ia + gd * ic;
    const float td = gc * ib + gd * id;
    out4[g * 4 + 0] = -(ia * ta + ib * tc);
    out4[g * 4 + 1] = -(ia * tb + ib * td);
    out4[g * 4 + 2] = -(ic * ta + id * tc);
    out4[g * 4 + 3] = -(ic * tb + id * td);
  }
}

/* --------------------------------------------------------------- ASM */

/* bandlimited_propagation_{forward,backward}_kernel with their host code
 * (bandlimited_propagation_cuda.cu:29-147,149-275) on split re/im and the
 * FX/FY grids, nx == ny.  adjoint != 0 selects phase = -distance*kz. */
void oracle_asm_spectral(const float* re, const float* im, const float* fxg, const float* fyg,
                         float* ore, float* oim, int nx, int ny, float wavelength,
                         float distance, float aperture, float pitch, int adjoint) {
  const float k = (float)(2.0 * 3.14159265358979323846 / (double)wavelength);
  const float x_size = pitch * (float)nx;
  const float y_size = pitch * (float)ny;
  const float fx_max = 1.0f / sqrtf((2.0f * distance * (1.0f / x_size)) * (2.0f * distance * (1.0f / x_size)) + 1.0f) / wavelength;
  const float fy_max = 1.0f / sqrtf((2.0f * distance * (1.0f / y_size)) * (2.0f * distance * (1.0f / y_size)) + 1.0f) / wavelength;
  const float offset_x = (float)nx / 2.0f - 0.5f;
  const float offset_y = (float)ny / 2.0f - 0.5f;
  const double two_pi = 2 * 3.14159265358979323846;
#pragma omp parallel for schedule(static)
  for (int idy = 0; idy < ny; ++idy)
    for (int idx = 0; idx < nx; ++idx) {
      const int64_t index = (int64_t)idy * nx + idx;
      const float fxv = fxg[index], fyv = fyg[index];
      const int within = (fabsf(fxv) < fx_max) && (fabsf(fyv) < fy_max);
      const float kz2 = (float)((double)(k * k) - (two_pi * (double)fxv) * (two_pi * (double)fxv) -
                                (two_pi * (double)fyv) * (two_pi * (double)fyv));
      float tr_re = 0.0f, tr_im = 0.0f;
      if (kz2 > 0.0f && within) {
        const float kz = sqrtf(kz2);
        const float ph = adjoint ? (-distance * kz) : (distance * kz);
        float sn, cs;
        sincosf(ph, &sn, &cs);
        tr_re = cs;
        tr_im = sn;
      }
      float ap = 1.0f;
      if (aperture > 0.0f) {
        const float x = (float)idx - offset_x;
        const float y = (float)idy - offset_y;
        ap = (x * x + y * y < aperture * aperture) ? 1.0f : 0.0f;
      }
      const float a = re[index], b = im[index];
      ore[index] = (a * tr_re - b * tr_im) * ap;
      oim[index] = (a * tr_im + b * tr_re) * ap;
    }
}

/* The scalar constants the ASM host code derives (for tests). */
void oracle_asm_consts(float wavelength, float distance, float pitch, int n, float* out4) {
  const float k = (float)(2.0 * 3.14159265358979323846 / (double)wavelength);
  const float x_size = pitch * (float)n;
  out4[0] = k;
  out4[1] = 1.0f / sqrtf((2.0f * distance * (1.0f / x_size)) * (2.0f * distance * (1.0f / x_size)) + 1.0f) / wavelength;
  out4[2] = (float)n / 2.0f - 0.5f;
  out4[3] = x_size;
}
