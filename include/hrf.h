/*
 * hrf.h — C ABI of the MI355X-native complex-valued wave rasterizer and
 * band-limited angular-spectrum (ASM) propagator.
 *
 * Every entry point takes raw device pointers, plain sizes and a hipStream_t
 * (passed as void*), returns an int status (HRF_OK == 0) and never throws.
 * On failure hrf_last_error() returns a message for the calling thread.
 * All kernels are enqueued on the given stream; the only host synchronisation
 * in the whole library is the pair/visible count read-back at the end of
 * hrf_raster_forward_prepare (the reference reads the same count back,
 * rasterizer_splat.cu:430-432).
 *
 * Layouts (all row-major, fp32 unless stated):
 *   cam_means (N,3), z_vals (N), quats (N,4) (r,x,y,z), scales (N,3),
 *   colours (N,C), phase (N,C), opacities (N), plane_probs (N,P),
 *   view_matrix (3,3) device memory, field (P,C,H,W) complex64 interleaved,
 *   final_T (P,H,W) f32, n_contrib (P,H,W) i32, point_list (K) i32,
 *   ranges (T,2) i32, visible (V) i64.  T = ceil(W/16)*ceil(H/16).
 */
#ifndef HRF_H
#define HRF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HRF_OK 0
#define HRF_ERR_INVALID 1   /* bad shape / argument */
#define HRF_ERR_HIP 2       /* a HIP / hipFFT call failed */
#define HRF_ERR_WORKSPACE 3 /* workspace too small */
#define HRF_ERR_OVERFLOW 4  /* pair count does not fit the int32 outputs */

/* Gaussians as passed to the rasterizer (post-activation values, device
 * pointers).  Mirrors the tensor arguments of Rasterizer::forward
 * (cuda_prop/cov3d_cuda/wave_rasterizer/rasterizer_splat.h:255-270). */
typedef struct hrf_gaussians {
  const float* cam_means;   /* (N,3) camera-space means */
  const float* z_vals;      /* (N)   depth used for culling and sorting */
  const float* quats;       /* (N,4) */
  const float* scales;      /* (N,3) */
  const float* colours;     /* (N,C) amplitudes */
  const float* phase;       /* (N,C) */
  const float* opacities;   /* (N) */
  const float* plane_probs; /* (N,P) */
  int64_t n;
  int32_t channels; /* C in 1..3 */
  int32_t planes;   /* P in 1..32 */
} hrf_gaussians;

/* Camera and image.  Mirrors the scalar arguments of Rasterizer::forward
 * (fx, fy, px, py, view_matrix, img_size=(W,H), near, far). */
typedef struct hrf_camera {
  float fx, fy, px, py;
  const float* view_matrix; /* (3,3) device pointer, used as W in cov2D */
  int32_t width, height;
  float near_plane, far_plane;
} hrf_camera;

const char* hrf_last_error(void);
/* Library version string ("hrf <major>.<minor> gfx950"). */
const char* hrf_version(void);

/* ---------------- rasterizer (replaces CudaRasterizer::Rasterizer) -------- */

/* Bytes of the per-Gaussian workspace ("geometry state") that must persist
 * from hrf_raster_forward_prepare to hrf_raster_forward_render.
 * Replaces GeometryState/CudaMemoryManager (rasterizer_splat.h:9-39,192-248). */
size_t hrf_raster_geom_workspace_size(int64_t n, int32_t channels, int32_t planes);

/* Bytes of the per-pair workspace ("binning state") for K pairs.
 * Replaces BinningState/ImageState (rasterizer_splat.h:64-94). */
size_t hrf_raster_binning_workspace_size(int64_t num_pairs, int32_t width, int32_t height);

/* Forward, phase 1: projection (means2D, J, Sigma, cov2D), culling, radius,
 * tile counts, depth ordering, offsets, visibility; reads back the pair
 * count K and the visible count V (one host sync).
 * Replaces Rasterizer::forward up to the K read-back
 * (rasterizer_splat.cu:324-432). */
int hrf_raster_forward_prepare(const hrf_gaussians* g, const hrf_camera* cam,
                               void* geom_ws, size_t geom_ws_bytes, void* stream,
                               int64_t* num_pairs, int64_t* num_visible);

/* Forward, phase 2: pair emission, stable tile sort, tile ranges and the
 * complex tile render.  Writes field, final_T, n_contrib, point_list (K),
 * ranges (T,2) and visible (V).  With K == 0 it writes the reference's
 * empty-scene outputs (rasterizer_splat.cu:434-449): zero field, final_T=1,
 * n_contrib=0, ranges=0; point_list and visible are not touched.
 * num_pairs and num_visible must be the counts hrf_raster_forward_prepare
 * returned for this geometry workspace (point_list holds num_pairs entries,
 * visible num_visible).  Other counts are rejected with HRF_ERR_INVALID
 * before anything is enqueued (the library keeps the counts of the last
 * prepare per workspace, for up to 256 workspaces); past that record, no
 * kernel writes more than num_pairs / num_visible entries whatever the
 * counts.  A count beyond 2^31 - 1 returns HRF_ERR_OVERFLOW.
 * Replaces rasterizer_splat.cu:451-547 and forward_splat.cu:101-289. */
int hrf_raster_forward_render(const hrf_gaussians* g, const hrf_camera* cam,
                              void* geom_ws, size_t geom_ws_bytes,
                              void* bin_ws, size_t bin_ws_bytes,
                              int64_t num_pairs, int64_t num_visible,
                              void* field, float* final_T, int32_t* n_contrib,
                              int32_t* point_list, int32_t* ranges, int64_t* visible,
                              void* plane_lists, size_t plane_lists_bytes,
                              void* stream);

/* Bytes of the optional plane member lists for K pairs on a W x H image
 * with P planes: P*K (gaussian, list position) int32 pairs (plane q's list
 * of tile t starts at q*K + ranges[t][0]), then, each from the next
 * 256-byte boundary, T*P int32 counts (tile-major) and the T*P (tile, plane)
 * ids t*P + q ordered by count, largest first (the backward's block order).
 * hrf_raster_forward_render fills the lists and counts (plane_lists
 * non-NULL) with each (tile, plane)'s members, in list order, over the
 * entries its compositing visited, that can reach alpha >= 1/255 in some
 * 8x8 quadrant of the tile (the quadrant mask rides in bits 28-31 of the
 * list position, so lists need N < 2^28); hrf_raster_backward given the same
 * buffer writes the block order from the counts and walks those lists
 * instead of filtering every tile list once per plane.  No
 * counterpart in the reference (its backward re-reads the whole tile list
 * per plane, backward_splat.cu:148-306). */
size_t hrf_raster_plane_lists_size(int64_t num_pairs, int32_t width, int32_t height,
                                   int32_t planes);

/* Bytes of workspace hrf_raster_backward needs. */
size_t hrf_raster_backward_workspace_size(int64_t n, int32_t channels, int32_t planes);

/* Backward: render backward (back-to-front recurrence) and the fused
 * geometry backward (means2D, cov2D, Jacobian, Sigma chains).
 * Outputs, all fully overwritten: grad_cam (N,3), grad_z (N) (always 0),
 * grad_quats (N,4), grad_scales (N,3), grad_colours (N,C), grad_phase (N,C),
 * grad_opacities (N), grad_plane_probs (N,P).
 * fwd_geom_ws (optional, may be NULL): the geometry workspace the forward of
 * these same inputs used, kept unchanged since; its render records are then
 * reused instead of recomputing the projection (the reference recomputes
 * means2D and cov2D, rasterizer_splat.cu:606-617).
 * plane_lists (optional, may be NULL): the plane member lists the forward of
 * these same inputs wrote (same point_list, ranges and n_contrib); the
 * backward writes their block-order words (the lists and counts are only
 * read).
 * Replaces Rasterizer::backward (rasterizer_splat.cu:551-684),
 * backward_splat.cu:78-417 and backward.cu. */
/* Queues the backward's prologue (clearing the per-Gaussian accumulators in
 * ws and forming the block order from the plane lists' counts) on `stream`
 * ahead of the backward, so that it can run beside other work (the
 * propagation adjoint) on another stream.  The next hrf_raster_backward on
 * the same ws, N, channels, planes, num_pairs and plane_lists waits for it
 * (an event recorded after it) instead of running it; with anything else
 * that call runs its own prologue.  The caller orders `stream` after the
 * forward that wrote plane_lists and after any earlier use of ws.  No
 * counterpart in the reference (its backward clears inside
 * Rasterizer::backward, rasterizer_splat.cu:551-684). */
int hrf_raster_backward_prepare(const hrf_gaussians* g, const hrf_camera* cam,
                                int64_t num_pairs, void* ws, size_t ws_bytes,
                                void* plane_lists, size_t plane_lists_bytes, void* stream);
int hrf_raster_backward(const hrf_gaussians* g, const hrf_camera* cam,
                        const void* grad_field, const float* final_T,
                        const int32_t* n_contrib, const int32_t* point_list,
                        const int32_t* ranges, int64_t num_pairs,
                        void* ws, size_t ws_bytes,
                        const void* fwd_geom_ws, size_t fwd_geom_ws_bytes,
                        void* plane_lists, size_t plane_lists_bytes,
                        float* grad_cam, float* grad_z, float* grad_quats,
                        float* grad_scales, float* grad_colours, float* grad_phase,
                        float* grad_opacities, float* grad_plane_probs,
                        void* stream);

/* ---------------- standalone geometry operators ----------------------------
 * The reference's separate autograd operators (cov3d_cuda module,
 * binding.cpp:14-25; python_import.py:53-281).  The rasterizer does not call
 * them (its projection and geometry backward are fused); they exist for
 * callers of compute_cov3d_cuda & co.  All tensors row-major fp32 on the
 * device; n Gaussians; outputs fully overwritten. */

/* Sigma = R S^2 R^T, cov3d (n,3,3).  Replaces compute_cov3d_forward
 * (wave_rasterizer/forward.cu:138-181). */
int hrf_cov3d_forward(const float* quats, const float* scales, int64_t n, float* cov3d,
                      void* stream);
/* grad_quats (n,4), grad_scales (n,3) from grad_cov3d (n,3,3).  Replaces
 * compute_cov3d_backward (wave_rasterizer/backward.cu:274-320). */
int hrf_cov3d_backward(const float* grad_cov3d, const float* quats, const float* scales,
                       int64_t n, float* grad_quats, float* grad_scales, void* stream);
/* Projection Jacobian (n,2,3), zero outside (near, far), clamp at
 * 1.3 * 0.5 * width / fx.  Replaces compute_jacobian_forward
 * (forward.cu:183-219). */
int hrf_jacobian_forward(const float* cam_means, int64_t n, float fx, float fy, int32_t width,
                         int32_t height, float near_plane, float far_plane, float* jacobian,
                         void* stream);
/* grad_cam (n,3) from grad_jacobian (n,2,3).  Replaces
 * compute_jacobian_backward (backward.cu:322-361). */
int hrf_jacobian_backward(const float* grad_jacobian, const float* cam_means, int64_t n,
                          float fx, float fy, int32_t width, int32_t height, float near_plane,
                          float far_plane, float* grad_cam, void* stream);
/* cov2D (n,2,2) = ((J W) Sigma) W^T J^T + 0.3 I and the saved J (n,2,3),
 * Sigma (n,3,3), W repeated (n,3,3), JW (n,2,3).  Replaces
 * compute_cov2d_forward (forward.cu:221-294). */
int hrf_cov2d_forward(const float* cam_means, const float* quats, const float* scales,
                      const float* view_matrix, int64_t n, float fx, float fy, int32_t width,
                      int32_t height, float near_plane, float far_plane, float* cov2d,
                      float* jacobian, float* cov3d, float* view_rep, float* jw, void* stream);
/* grad_cam (n,3), grad_quats (n,4), grad_scales (n,3) from grad_cov2d
 * (n,2,2), using the saved J, Sigma, W, JW as given (view_matrix is unused,
 * as in the reference).  Replaces compute_cov2d_backward
 * (backward.cu:363-450). */
int hrf_cov2d_backward(const float* grad_cov2d, const float* cam_means, const float* quats,
                       const float* scales, const float* view_matrix, const float* jacobian,
                       const float* cov3d, const float* view_rep, const float* jw, int64_t n,
                       float fx, float fy, int32_t width, int32_t height, float near_plane,
                       float far_plane, float* grad_cam, float* grad_quats, float* grad_scales,
                       void* stream);
/* means2D (n,2) = (fx*(-x/z)+px, fy*(-y/z)+py), (1e6, 1e6) outside (near,
 * far).  Replaces compute_means2d_forward (forward.cu:358-394). */
int hrf_means2d_forward(const float* cam_means, int64_t n, float fx, float fy, float px,
                        float py, float near_plane, float far_plane, float* means2d,
                        void* stream);
/* grad_cam (n,3) from grad_means2d (n,2).  Replaces compute_means2d_backward
 * (backward.cu:545-585). */
int hrf_means2d_backward(const float* grad_means2d, const float* cam_means, int64_t n, float fx,
                         float fy, float px, float py, float near_plane, float far_plane,
                         float* grad_cam, void* stream);
/* (n,2,2) inverse.  Replaces invert_cov2d_forward (forward.cu:396-432). */
int hrf_invert_cov2d_forward(const float* cov2d, int64_t n, float* cov2d_inverse, void* stream);
/* grad_cov2d = -(A^-1 G A^-1).  Replaces invert_cov2d_backward
 * (backward.cu:587-627). */
int hrf_invert_cov2d_backward(const float* grad_inverse, const float* cov2d, int64_t n,
                              float* grad_cov2d, void* stream);

/* ---------------- band-limited ASM (replaces cuda_modules) ---------------- */

/* Spectral multiply on a pre-shifted (fftshift) spectrum, reading the
 * frequency grids, exactly as bound by cuda_modules.bandlimited_propagation_
 * forward(re, im, FX, FY, wavelength, distance, aperture, pitch)
 * (cuda_prop/cpp/module_def.cpp:4-13,55-56; cuda_prop/cpp/bandlimited_
 * propagation.cpp:34-54).  nx = rows, ny = cols; only nx == ny is defined. */
int hrf_asm_spectral_forward(const float* re, const float* im,
                             const float* fx_grid, const float* fy_grid,
                             float* out_re, float* out_im, int32_t nx, int32_t ny,
                             float wavelength, float distance, float aperture,
                             float pixel_pitch, void* stream);

/* Adjoint spectral multiply (conjugate transfer function).  field_re/im are
 * accepted for signature parity and unused, as in the reference
 * (cuda_prop/cpp/bandlimited_propagation.cpp:57-80). */
int hrf_asm_spectral_backward(const float* grad_re, const float* grad_im,
                              const float* field_re, const float* field_im,
                              const float* fx_grid, const float* fy_grid,
                              float* out_re, float* out_im, int32_t nx, int32_t ny,
                              float wavelength, float distance, float aperture,
                              float pixel_pitch, void* stream);

/* Workspace for the whole-propagation entry points below: M = 2*S.
 * Grids with M in {128, 160, 192, 512, 1024, 1600, 2016, 2048} run the
 * fused hand-written LDS-FFT kernels (row pass with the zero pad, column
 * pass with the transfer-function multiply summed over planes and the row
 * crop, inverse row pass with the column crop and 1/M^2); other even sizes
 * run the same arithmetic around hipFFT transforms. */
size_t hrf_asm_workspace_size(int32_t planes, int32_t channels, int32_t size);

/* One field (H,W) c64 -> (S,S) c64: centred zero pad to (2S,2S), FFT,
 * transfer function x band-limit x aperture, inverse FFT (1/M^2), centred
 * crop.  Replaces BandlimitedPropagationFunction.forward
 * (cuda_prop/python_function.py:111-163).  pixel_pitch is double because the
 * reference builds its frequency grid with torch.fft.fftfreq(d=pitch) from a
 * Python float. */
int hrf_asm_forward(const void* field, int32_t height, int32_t width, int32_t size,
                    float wavelength, double pixel_pitch, float distance,
                    float aperture, void* out, void* ws, size_t ws_bytes, void* stream);

/* Exact adjoint of hrf_asm_forward: (S,S) c64 -> (H,W) c64.  Replaces
 * BandlimitedPropagationFunction.backward (python_function.py:166-218). */
int hrf_asm_adjoint(const void* grad_out, int32_t height, int32_t width, int32_t size,
                    float wavelength, double pixel_pitch, float distance,
                    float aperture, void* grad_field, void* ws, size_t ws_bytes,
                    void* stream);

/* All planes and wavelengths at once: fields (P,C,H,W) c64 ->
 * hologram (C,S,S) c64 with hologram[c] = sum_p propagate(fields[p,c],
 * wavelengths[c], distances[p]).  wavelengths (C) and distances (P) are host
 * arrays of the per-call propagation distances.  Replaces the per-(p,c) loop
 * and the Python sum in Scene.splat (model.py:1251-1272). */
int hrf_asm_multiplane_forward(const void* fields, int32_t planes, int32_t channels,
                               int32_t height, int32_t width, int32_t size,
                               const float* wavelengths, const float* distances,
                               double pixel_pitch, float aperture, void* hologram,
                               void* ws, size_t ws_bytes, void* stream);

/* Adjoint of hrf_asm_multiplane_forward: grad hologram (C,S,S) ->
 * grad fields (P,C,H,W). */
int hrf_asm_multiplane_adjoint(const void* grad_hologram, int32_t planes,
                               int32_t channels, int32_t height, int32_t width,
                               int32_t size, const float* wavelengths,
                               const float* distances, double pixel_pitch,
                               float aperture, void* grad_fields, void* ws,
                               size_t ws_bytes, void* stream);

/* One field per wavelength, many distances: fields (C,H,W) c64 ->
 * out (D,C,S,S) c64 with out[d,c] = propagate(fields[c], wavelengths[c],
 * distances[d]).  Each channel is transformed once and shared by all D
 * distances (C + D*C transforms instead of 2*D*C).  Replaces the
 * per-(distance, wavelength) BandlimitedPropagation calls of the
 * propagation microbench (python_function.py:220-226).  Any even size
 * (hipFFT transforms). */
size_t hrf_asm_multidistance_workspace_size(int32_t channels, int32_t size);
int hrf_asm_multidistance_forward(const void* fields, int32_t num_distances,
                                  int32_t channels, int32_t height, int32_t width,
                                  int32_t size, const float* wavelengths,
                                  const float* distances, double pixel_pitch,
                                  float aperture, void* out, void* ws, size_t ws_bytes,
                                  void* stream);
/* Adjoint: grad out (D,C,S,S) -> grad fields (C,H,W) = sum over d of the
 * single-distance adjoints, summed in the spectral domain (D*C + C
 * transforms). */
int hrf_asm_multidistance_adjoint(const void* grad_out, int32_t num_distances,
                                  int32_t channels, int32_t height, int32_t width,
                                  int32_t size, const float* wavelengths,
                                  const float* distances, double pixel_pitch,
                                  float aperture, void* grad_fields, void* ws,
                                  size_t ws_bytes, void* stream);

/* Releases cached hipFFT plans and FFT twiddle tables (optional). */
void hrf_release_caches(void);

/* ---------------- render preprocess (Scene.render's glue) -----------------
 * The caller-side steps between the model's parameters and the rasterizer
 * (Scene.render, model.py:1365-1402; Scene.splat's world-to-view transform,
 * model.py:1161-1162): X_cam = X_world @ R + T, keep near < z < far and
 * z >= 0 (model.py:1382-1385,1121-1125), ascending stable depth order, the
 * gathers, and Gaussians.apply_activations (model.py:594-608): exp(scales),
 * F.normalize(quats), phase mod 2*pi, sigmoid(opacities), one_hot(argmax)
 * plane probabilities (STEFunction, model.py:41-56).  The reference sorts
 * with torch.sort (order of equal depths unspecified); here ties keep the
 * index order. */
typedef struct hrf_scene_params {
  const float* means;         /* (N,3) world-space means */
  const float* pre_quats;     /* (N,4) */
  const float* pre_scales;    /* (N,3) log scales */
  const float* colours;       /* (N,C) */
  const float* pre_phase;     /* (N,C) */
  const float* pre_opacities; /* (N) */
  const float* pre_plane;     /* (N,P) plane-assignment logits */
  int64_t n;
  int32_t channels; /* C >= 1 */
  int32_t planes;   /* P in 1..32 */
} hrf_scene_params;

/* Gradients of the M selected rows (the outputs of hrf_preprocess_forward). */
typedef struct hrf_selected_grads {
  const float* cam;         /* (M,3) */
  const float* z;           /* (M), NULL = zero */
  const float* quats;       /* (M,4) */
  const float* scales;      /* (M,3) */
  const float* colours;     /* (M,C) */
  const float* phase;       /* (M,C) */
  const float* opacities;   /* (M) */
  const float* plane_probs; /* (M,P) */
} hrf_selected_grads;

/* Gradients of the N parameter rows; fully overwritten (rows that were not
 * selected get zeros). */
typedef struct hrf_param_grads {
  float* means;
  float* pre_quats;
  float* pre_scales;
  float* colours;
  float* pre_phase;
  float* pre_opacities;
  float* pre_plane;
} hrf_param_grads;

/* Workspace of hrf_preprocess_select / _forward / _backward for N Gaussians
 * with C colour channels and P planes; it carries the selection from
 * _select to _forward (the backward needs nothing from them). */
size_t hrf_preprocess_workspace_size(int64_t n, int32_t channels, int32_t planes);

/* Camera transform, selection and depth order; returns the selected count M
 * (one host sync, as the reference's torch.where / masked_select).  R (3,3)
 * row-major and T (3) are device pointers (camera.R[0], camera.T[0]).
 * Replaces model.py:1377-1388. */
int hrf_preprocess_select(const hrf_scene_params* params, const float* R, const float* T,
                          float near_plane, float far_plane, void* ws, size_t ws_bytes,
                          void* stream, int64_t* num_selected);

/* Gathers and activations of the M selected Gaussians, in depth order:
 * cam_means (M,3), z_vals (M), quats (M,4), scales (M,3), colours (M,C),
 * phase (M,C), opacities (M), plane_probs (M,P) and idxs (M) int64, the
 * parameter row of each.  Replaces model.py:1389-1402 and 1161-1162. */
int hrf_preprocess_forward(const hrf_scene_params* params, const float* R, const float* T,
                           const void* ws, size_t ws_bytes, int64_t num_selected,
                           float* cam_means, float* z_vals, float* quats, float* scales,
                           float* colours, float* phase, float* opacities,
                           float* plane_probs, int64_t* idxs, void* stream);

/* Backward of hrf_preprocess_forward: the gradients of its outputs -> the
 * parameter gradients (autograd of the reference's gathers and activations;
 * the plane logits get grad * softmax(logits / 0.001), STEFunction.backward,
 * model.py:50-56).  ws: hrf_preprocess_workspace_size bytes. */
int hrf_preprocess_backward(const hrf_scene_params* params, const float* R,
                            const int64_t* idxs, int64_t num_selected,
                            const hrf_selected_grads* grads, const hrf_param_grads* out,
                            void* ws, size_t ws_bytes, void* stream);

/* ---------------- loss-side reconstruction (utils/propagator.py:548-636) ---
 * propagator._reconstruct_impl: for each frame f and channel c with laser
 * power w = laser_powers[f][c] != 0 (K such pairs, listed as frames[k],
 * channels[k], powers[k], scales[k] = phase_scale[c]), the hologram field
 * w a_c e^{i s phi_f}, propagated to every depth (the multi-distance ASM
 * entry points above) and its intensity |u|^2.  amplitude (C, hw), phase
 * (F, hw) float32; fields and gradients complex64 interleaved. */

/* fields (K, hw) from the amplitude and phase maps (generate_complex_field,
 * propagator.py:605-609). */
int hrf_recon_fields(const float* amplitude, const float* phase, int32_t F, int32_t C,
                     int64_t hw, const int32_t* frames, const int32_t* channels,
                     const float* powers, const float* scales, int32_t K, void* fields,
                     void* stream);

/* intensity[i] = |field[i]|^2 (calculate_amplitude(.)**2, :626). */
int hrf_recon_intensity(const void* field, int64_t n, float* intensity, void* stream);

/* grad_field = 2 grad_intensity field (the backward of |u|^2). */
int hrf_recon_intensity_backward(const void* field, const float* grad_intensity, int64_t n,
                                 void* grad_field, void* stream);

/* Backward of hrf_recon_fields: grad_amplitude (C, hw) and grad_phase
 * (F, hw), summed over the pairs (fully overwritten). */
int hrf_recon_fields_backward(const float* amplitude, const float* phase, int32_t F, int32_t C,
                              int64_t hw, const int32_t* frames, const int32_t* channels,
                              const float* powers, const float* scales, int32_t K,
                              const void* grad_fields, float* grad_amplitude,
                              float* grad_phase, void* stream);

/* ---------------- optimizer step (train.py:319-324) -----------------------
 * The reference clips the global gradient norm (torch.nn.utils.clip_grad_norm_
 * (parameters, 1.0)) and then steps Adan (utils/optimizer.py:288-466, the
 * foreach path _multi_tensor_adan, :538-589) over the seven parameter
 * tensors.  Here: one pass for the norm (fixed-order partial sums, the clip
 * coefficient formed on the device), one pass for the update. */

/* Scratch of hrf_grad_norm: one float per 2048-element chunk of each tensor
 * plus one. */
size_t hrf_grad_norm_workspace_size(const int64_t* numels, int32_t num_tensors);

/* total_norm = ||all gradients||_2 and clip_coef = min(max_norm /
 * (total_norm + 1e-6), 1) (NaN propagates), both device floats (either may
 * be NULL), as clip_grad_norm_ forms them (torch/nn/utils/clip_grad.py).
 * grads: host array of device pointers.  Replaces the norm half of
 * train.py:319. */
int hrf_grad_norm(const float* const* grads, const int64_t* numels, int32_t num_tensors,
                  float max_norm, float* total_norm, float* clip_coef, void* ws,
                  size_t ws_bytes, void* stream);

/* hrf_grad_norm without a workspace: the partial sums live in a static
 * device array of the library (65536 floats, 256 KiB per GPU, held until the
 * process ends), so this entry point allocates nothing and calls no
 * allocating routine.  No counterpart in the reference: it is for callers
 * that cannot allocate (code under HIP graph capture, tight training or
 * serving loops, harnesses that forbid allocation).  At most 65536 * 2048 =
 * 134217728 gradient elements in total (HRF_ERR_WORKSPACE beyond).  Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams or host threads) race and must be ordered by the caller.
 * Same results as hrf_grad_norm (same kernels, same summation order).  The
 * first call on a device looks up the array's device address
 * (hipGetSymbolAddress, which allocates nothing); a caller that captures the
 * call into a HIP graph makes one call on that device before capturing.
 * Stage tracing (hrf_trace_enable) does not time this entry point. */
int hrf_grad_norm_static(const float* const* grads, const int64_t* numels, int32_t num_tensors,
                         float max_norm, float* total_norm, float* clip_coef, void* stream);

/* grads *= *coef (device scalar): the rescaling half of clip_grad_norm_. */
int hrf_scale_grads(float* const* grads, const int64_t* numels, int32_t num_tensors,
                    const float* coef, void* stream);

typedef struct hrf_adan_tensor {
  float* param;        /* updated in place */
  float* grad;         /* read; left holding the gradient times the scales */
  float* exp_avg;      /* Adan state, as the reference names it */
  float* exp_avg_sq;
  float* exp_avg_diff;
  float* neg_pre_grad;
  int64_t numel;
  double lr;           /* the tensor's group learning rate */
  int64_t step;        /* the group's step count for this step (>= 1) */
  int32_t init_neg_pre_grad; /* 1: neg_pre_grad = -grad first (step 1 or no
                                 state, optimizer.py:439-441) */
} hrf_adan_tensor;

typedef struct hrf_adan_config {
  double beta1, beta2, beta3; /* (0.98, 0.92, 0.99) in the reference */
  double eps;                 /* 1e-8 */
  double weight_decay;        /* 0 */
  double clip_global_grad_norm; /* Adan's own max_grad_norm clip (1 when 0) */
  int32_t no_prox;
} hrf_adan_config;

/* One Adan step over all tensors (_multi_tensor_adan, op for op in float32,
 * scalars formed in double on the host).  grad_scale (device float, may be
 * NULL) multiplies the gradients first: passing hrf_grad_norm's clip_coef
 * folds clip_grad_norm_'s rescaling into this pass. */
int hrf_adan_step(const hrf_adan_tensor* tensors, int32_t num_tensors,
                  const hrf_adan_config* cfg, const float* grad_scale, void* stream);

/* ---------------- training-loop helpers of the cov3d_cuda module ----------
 * The two remaining names python_import.py exports (utils/data_utils.py:20
 * and utils/optimizer.py:21 import them). */

/* SSIM map of two (C,H,W) float images, 11x11 Gaussian window (sigma 1.5)
 * with zero padding, written to ssim_map (C,H,W); c1, c2 the stabilising
 * constants (0.01^2, 0.03^2 in the reference).  Replaces fusedssim
 * (cuda_prop/cov3d_cuda/conv.cu:935-1002,1138-1166) behind fast_ssim
 * (python_import.py:43-58,449-454), which supports C = 3 only. */
int hrf_ssim_map(const float* img1, const float* img2, int32_t channels, int32_t height,
                 int32_t width, float c1, float c2, float* ssim_map, void* stream);

/* grad_img1 (C,H,W) = d(sum grad_map * ssim_map)/d img1 (img2 gets no
 * gradient, as in the reference).  Replaces fusedssim_backward
 * (conv.cu:1011-1135,1168-1197). */
int hrf_ssim_backward(const float* img1, const float* img2, const float* grad_map,
                      int32_t channels, int32_t height, int32_t width, float c1, float c2,
                      float* grad_img1, void* stream);

/* Sparse Adam step over the visible rows, no bias correction: param,
 * exp_avg, exp_avg_sq (batch, rows, cols); grad (batch, num_visible, cols),
 * the visible rows' gradients in the order of visible (num_visible) int64
 * row indices.  Rows outside [0, rows) are skipped.  Replaces adamUpdate
 * (cuda_prop/cov3d_cuda/spadam.cu:8-55) behind sparse_adam_update
 * (python_import.py:457-460). */
int hrf_sparse_adam_update(float* param, const float* grad, float* exp_avg, float* exp_avg_sq,
                           const int64_t* visible, int64_t batch, int64_t rows, int64_t cols,
                           int64_t num_visible, float lr, float beta1, float beta2, float eps,
                           void* stream);

/* ---------------- stage tracing (no counterpart in the reference, which
 * prints per-phase CUDA event times from train.py:263-344) ---------------- */

/* Enables (1) or disables (0) stage tracing.  While enabled, every kernel
 * stage of the calls above is bracketed by a pair of hipEvents recorded on
 * the caller's stream. */
int hrf_trace_enable(int on);
/* Restricts tracing to one stage (NULL or "" traces every stage).  Each
 * traced stage adds two event records to the caller's stream, which costs
 * queue time: trace a single stage while measuring throughput. */
int hrf_trace_only(const char* stage);
/* Clears all recorded stage events. */
void hrf_trace_reset(void);
/* Waits for the recorded events of `stage` and returns the number of
 * launches and their summed duration in milliseconds since the last reset.
 * Stages: project, depth_sort, scan, emit, tile_sort, ranges, render_fwd,
 * render_bwd, geom_bwd; fused propagation: asm_rows_in, asm_col_fwd,
 * asm_col_adj, asm_rows_out; hipFFT propagation: asm_pad, asm_fft,
 * asm_mac_fwd, asm_mac_adj, asm_crop; preprocess: pre_select, pre_gather,
 * pre_backward. */
int hrf_trace_read(const char* stage, int64_t* launches, double* total_ms);

#ifdef __cplusplus
}
#endif

#endif /* HRF_H */
