"""Python face of the CPU oracle — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the checker.  The product package
never imports it.

It wraps ``liboracle_hrf.so`` (``hrf_oracle.c``, a literal C restatement of
the reference CUDA code) and composes the reference's ASM propagation
(``cuda_prop/python_function.py:111-218``) from that spectral kernel and
numpy's FFT (pocketfft, computed in double precision).

What independently checks each function (closed forms, brute force,
float64 restatements, finite differences, a brute-force DFT, invariants) is
in ``tests/test_oracle_pinning.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_hrf.so")
# HRF_ORACLE_LIB selects another build of the same source (the sanitizer
# build, `make sanitized`); the default is the optimised library.
_ALT_LIB = os.environ.get("HRF_ORACLE_LIB")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float


def build() -> str:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    src = os.path.join(_HERE, "hrf_oracle.c")
    if _ALT_LIB:
        _lib = _bind(ctypes.CDLL(_ALT_LIB))
        return _lib
    if not os.path.exists(_LIB_PATH) or (
        os.path.exists(src) and os.path.getmtime(src) > os.path.getmtime(_LIB_PATH)
    ):
        build()
    _lib = _bind(ctypes.CDLL(_LIB_PATH))
    return _lib


def _bind(L):
    L.oracle_cov3d.argtypes = [_f32p, _f32p, _f32p]
    L.oracle_project.argtypes = [_i64, _f32p, _f32p, _f32p, _f32p, _flt, _flt, _flt, _flt,
                                 _int, _int, _flt, _flt, _f32p, _f32p, _f32p, _f32p, _f32p]
    L.oracle_preprocess.argtypes = [_i64, _f32p, _f32p, _f32p, _int, _int, _flt, _flt,
                                    _i32p, _u32p, _u32p]
    L.oracle_count_pairs.argtypes = [_i64, _u32p]
    L.oracle_count_pairs.restype = _i64
    L.oracle_bin.argtypes = [_i64, _f32p, _u32p, _u32p, _int, _int, _i64, _i32p, _i32p]
    L.oracle_render_forward.argtypes = [_int, _int, _int, _int, _i32p, _i32p, _f32p, _f32p,
                                        _f32p, _f32p, _f32p, _f32p, _f32p, _flt, _flt,
                                        _f32p, _f32p, _i32p, ctypes.c_void_p]
    L.oracle_render_backward.argtypes = [_i64, _int, _int, _int, _int, _i32p, _i32p, _f32p,
                                         _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i32p,
                                         _f32p, _f64p, _f64p, _f64p, _f64p, _f64p, _f64p,
                                         ctypes.c_void_p]
    L.oracle_geom_backward.argtypes = [_i64, _f32p, _f32p, _f32p, _f32p, _flt, _flt, _int,
                                       _int, _flt, _flt, _f32p, _f32p, _f32p, _f32p, _f32p,
                                       _f32p, _f32p]
    L.oracle_cov3d_backward.argtypes = [_i64, _f32p, _f32p, _f32p, _f32p, _f32p]
    L.oracle_jacobian_backward.argtypes = [_i64, _f32p, _f32p, _flt, _flt, _int, _int, _flt,
                                           _flt, _f32p]
    L.oracle_cov2d_backward.argtypes = [_i64, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                        _f32p, _flt, _flt, _int, _int, _flt, _flt, _f32p,
                                        _f32p, _f32p]
    L.oracle_means2d_backward.argtypes = [_i64, _f32p, _f32p, _flt, _flt, _flt, _flt, _f32p]
    L.oracle_invert_cov2d.argtypes = [_i64, _f32p, _f32p]
    L.oracle_invert_cov2d_backward.argtypes = [_i64, _f32p, _f32p, _f32p]
    L.oracle_asm_spectral.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _int, _int,
                                      _flt, _flt, _flt, _flt, _int]
    L.oracle_asm_consts.argtypes = [_flt, _flt, _flt, _int, _f32p]
    return L


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


@dataclass
class Camera:
    fx: float
    fy: float
    px: float
    py: float
    view: np.ndarray  # (3,3) float32
    width: int
    height: int
    near: float = 1.0
    far: float = 1000.0


@dataclass
class Gaussians:
    cam_means: np.ndarray  # (N,3)
    z: np.ndarray  # (N,)
    quats: np.ndarray  # (N,4)
    scales: np.ndarray  # (N,3)
    colours: np.ndarray  # (N,C)
    phase: np.ndarray  # (N,C)
    opac: np.ndarray  # (N,)
    pprobs: np.ndarray  # (N,P)

    @property
    def n(self):
        return int(self.cam_means.shape[0])

    @property
    def C(self):
        return int(self.colours.shape[1])

    @property
    def P(self):
        return int(self.pprobs.shape[1])


def cov3d(quats, scales):
    L = lib()
    n = quats.shape[0]
    out = np.zeros((n, 9), np.float32)
    q = _f32(quats)
    s = _f32(scales)
    for g in range(n):
        o = np.zeros(9, np.float32)
        L.oracle_cov3d(q[g], s[g], o)
        out[g] = o
    return out.reshape(n, 3, 3)


def project(g: Gaussians, cam: Camera):
    """means2D (N,2), J (N,2,3), Sigma (N,3,3), JW (N,2,3), cov2D (N,4)."""
    L = lib()
    n = g.n
    m = np.zeros((n, 2), np.float32)
    J = np.zeros((n, 6), np.float32)
    S = np.zeros((n, 9), np.float32)
    JW = np.zeros((n, 6), np.float32)
    c2 = np.zeros((n, 4), np.float32)
    L.oracle_project(n, _f32(g.cam_means), _f32(g.quats), _f32(g.scales), _f32(cam.view),
                     cam.fx, cam.fy, cam.px, cam.py, cam.width, cam.height, cam.near, cam.far,
                     m, J, S, JW, c2)
    return dict(means2d=m, J=J.reshape(n, 2, 3), sigma=S.reshape(n, 3, 3),
                JW=JW.reshape(n, 2, 3), cov2d=c2)


def preprocess(means2d, cov2d, z, cam: Camera):
    L = lib()
    n = means2d.shape[0]
    radii = np.zeros(n, np.int32)
    tiles = np.zeros(n, np.uint32)
    rect = np.zeros((n, 4), np.uint32)
    L.oracle_preprocess(n, _f32(means2d), _f32(cov2d), _f32(z), cam.width, cam.height,
                        cam.near, cam.far, radii, tiles, rect)
    return radii, tiles, rect


def bin_pairs(z, tiles, rect, cam: Camera):
    L = lib()
    n = z.shape[0]
    k = int(L.oracle_count_pairs(n, np.ascontiguousarray(tiles, np.uint32)))
    gx = (cam.width + 15) // 16
    gy = (cam.height + 15) // 16
    pl = np.zeros(max(k, 1), np.int32)
    ranges = np.zeros((gx * gy, 2), np.int32)
    L.oracle_bin(n, _f32(z), np.ascontiguousarray(tiles, np.uint32),
                 np.ascontiguousarray(rect, np.uint32), cam.width, cam.height, k, pl, ranges)
    return pl[:k], ranges


def _tile_mask(mask, cam: Camera):
    """(uint8 array kept alive, its address) for an optional per-tile mask."""
    if mask is None:
        return None, None
    T = ((cam.width + 15) // 16) * ((cam.height + 15) // 16)
    m = np.ascontiguousarray(mask, dtype=np.uint8)
    if m.shape != (T,):
        raise ValueError(f"tile mask must have {T} entries, got {m.shape}")
    return m, m.ctypes.data


def render_forward(g: Gaussians, cam: Camera, means2d, cov2d, point_list, ranges,
                   tile_mask=None):
    """Field (P,C,H,W), final_T and n_contrib (P,H,W); with tile_mask only the
    selected tiles' pixels are rendered (the rest stay 0)."""
    L = lib()
    keep, mptr = _tile_mask(tile_mask, cam)
    P, C, H, W = g.P, g.C, cam.height, cam.width
    field = np.zeros((P, C, H, W, 2), np.float32)
    fT = np.zeros((P, H, W), np.float32)
    nc = np.zeros((P, H, W), np.int32)
    pl = np.ascontiguousarray(point_list if len(point_list) else np.zeros(1), np.int32)
    L.oracle_render_forward(W, H, P, C, np.ascontiguousarray(ranges, np.int32), pl,
                            _f32(means2d), _f32(cov2d), _f32(g.z), _f32(g.colours),
                            _f32(g.phase), _f32(g.opac), _f32(g.pprobs), cam.near, cam.far,
                            field, fT, nc, mptr)
    del keep
    return field[..., 0] + 1j * field[..., 1], fT, nc


def render_backward(g: Gaussians, cam: Camera, means2d, cov2d, point_list, ranges, final_T,
                    n_contrib, grad_field, tile_mask=None):
    """Render-backward accumulators (float64); with tile_mask only the
    selected tiles' pixels contribute."""
    L = lib()
    keep, mptr = _tile_mask(tile_mask, cam)
    n, P, C, H, W = g.n, g.P, g.C, cam.height, cam.width
    gf = np.ascontiguousarray(
        np.stack([grad_field.real, grad_field.imag], axis=-1), dtype=np.float32)
    out = dict(means2d=np.zeros((n, 2)), cov2d=np.zeros((n, 4)), colours=np.zeros((n, C)),
               phase=np.zeros((n, C)), opac=np.zeros(n), plane=np.zeros((n, P)))
    pl = np.ascontiguousarray(point_list if len(point_list) else np.zeros(1), np.int32)
    L.oracle_render_backward(n, W, H, P, C, np.ascontiguousarray(ranges, np.int32), pl,
                             _f32(means2d), _f32(cov2d), _f32(g.colours), _f32(g.phase),
                             _f32(g.opac), _f32(g.pprobs), _f32(final_T),
                             np.ascontiguousarray(n_contrib, np.int32), gf, out["means2d"],
                             out["cov2d"], out["colours"], out["phase"], out["opac"],
                             out["plane"], mptr)
    del keep
    return out


def geom_backward(g: Gaussians, cam: Camera, grad_means2d, grad_cov2d, want_links=False):
    L = lib()
    n = g.n
    gc = np.zeros((n, 3), np.float32)
    gq = np.zeros((n, 4), np.float32)
    gs = np.zeros((n, 3), np.float32)
    dsig = np.zeros((n, 9), np.float32)
    dJ = np.zeros((n, 6), np.float32)
    L.oracle_geom_backward(n, _f32(g.cam_means), _f32(g.quats), _f32(g.scales), _f32(cam.view),
                           cam.fx, cam.fy, cam.width, cam.height, cam.near, cam.far,
                           _f32(grad_means2d), _f32(grad_cov2d), gc, gq, gs, dsig, dJ)
    if want_links:
        return gc, gq, gs, dsig.reshape(n, 3, 3), dJ.reshape(n, 2, 3)
    return gc, gq, gs


# ---------------------------------------------- standalone geometry operators
# (the reference's compute_*_{forward,backward}, binding.cpp:14-25)

def cov3d_forward(quats, scales):
    """compute_cov3d_forward (forward.cu:138-181): (N,3,3)."""
    L = lib()
    q, s = _f32(quats), _f32(scales)
    out = np.zeros((q.shape[0], 9), np.float32)
    for i in range(q.shape[0]):
        L.oracle_cov3d(q[i], s[i], out[i])
    return out.reshape(-1, 3, 3)


def cov3d_backward(grad, quats, scales):
    """compute_cov3d_backward (backward.cu:274-320)."""
    n = quats.shape[0]
    gq = np.zeros((n, 4), np.float32)
    gs = np.zeros((n, 3), np.float32)
    lib().oracle_cov3d_backward(n, _f32(grad).reshape(n, 9), _f32(quats), _f32(scales), gq, gs)
    return gq, gs


def jacobian_backward(grad, cam_means, fx, fy, W, H, near, far):
    """compute_jacobian_backward (backward.cu:322-361)."""
    n = cam_means.shape[0]
    out = np.zeros((n, 3), np.float32)
    lib().oracle_jacobian_backward(n, _f32(grad).reshape(n, 6), _f32(cam_means), fx, fy, W, H,
                                   near, far, out)
    return out


def cov2d_forward(g: Gaussians, cam: Camera):
    """compute_cov2d_forward (forward.cu:221-294): cov2D, J, Sigma, W rep, JW."""
    pr = project(g, cam)
    n = g.n
    W = np.broadcast_to(_f32(cam.view).reshape(1, 3, 3), (n, 3, 3)).copy()
    return pr["cov2d"].reshape(n, 2, 2), pr["J"], pr["sigma"], W, pr["JW"]


def cov2d_backward(grad, cam_means, quats, scales, J, sig, W, JW, fx, fy, Wd, Hd, near, far):
    """compute_cov2d_backward (backward.cu:363-450) on the saved intermediates."""
    n = cam_means.shape[0]
    gc = np.zeros((n, 3), np.float32)
    gq = np.zeros((n, 4), np.float32)
    gs = np.zeros((n, 3), np.float32)
    lib().oracle_cov2d_backward(n, _f32(grad).reshape(n, 4), _f32(cam_means), _f32(quats),
                                _f32(scales), _f32(J).reshape(n, 6), _f32(sig).reshape(n, 9),
                                _f32(W).reshape(n, 9), _f32(JW).reshape(n, 6), fx, fy, Wd, Hd,
                                near, far, gc, gq, gs)
    return gc, gq, gs


def means2d_backward(grad, cam_means, fx, fy, near, far):
    """compute_means2d_backward (backward.cu:545-585)."""
    n = cam_means.shape[0]
    out = np.zeros((n, 3), np.float32)
    lib().oracle_means2d_backward(n, _f32(grad), _f32(cam_means), fx, fy, near, far, out)
    return out


def invert_cov2d(cov):
    """invert_cov2d_forward (forward.cu:396-432)."""
    n = cov.shape[0]
    out = np.zeros((n, 4), np.float32)
    lib().oracle_invert_cov2d(n, _f32(cov).reshape(n, 4), out)
    return out.reshape(n, 2, 2)


def invert_cov2d_backward(grad, cov):
    """invert_cov2d_backward (backward.cu:587-627)."""
    n = cov.shape[0]
    out = np.zeros((n, 4), np.float32)
    lib().oracle_invert_cov2d_backward(n, _f32(grad).reshape(n, 4), _f32(cov).reshape(n, 4), out)
    return out.reshape(n, 2, 2)


def visible_indices(g: Gaussians, cam: Camera):
    z = g.cam_means[:, 2]
    return np.nonzero((z > 0.2) & (z > cam.near) & (z < cam.far))[0].astype(np.int64)


def rasterize_forward(g: Gaussians, cam: Camera):
    """Full SplatTileCuda forward: field (P,C,H,W) c64 + forward_info."""
    pr = project(g, cam)
    radii, tiles, rect = preprocess(pr["means2d"], pr["cov2d"], g.z, cam)
    pl, ranges = bin_pairs(g.z, tiles, rect, cam)
    K = len(pl)
    if K == 0:
        P, C, H, W = g.P, g.C, cam.height, cam.width
        return dict(field=np.zeros((P, C, H, W), np.complex64), final_T=np.ones((P, H, W), np.float32),
                    n_contrib=np.zeros((P, H, W), np.int32), point_list=np.zeros(1, np.int32),
                    ranges=ranges, visible=np.zeros(0, np.int64), K=0, proj=pr, radii=radii,
                    tiles=tiles, rect=rect)
    field, fT, nc = render_forward(g, cam, pr["means2d"], pr["cov2d"], pl, ranges)
    return dict(field=field.astype(np.complex64), final_T=fT, n_contrib=nc, point_list=pl,
                ranges=ranges, visible=visible_indices(g, cam), K=K, proj=pr, radii=radii,
                tiles=tiles, rect=rect)


def rasterize_backward(g: Gaussians, cam: Camera, fwd, grad_field):
    """Full Rasterizer::backward: the 8 gradients (float32)."""
    pr = fwd["proj"]
    rb = render_backward(g, cam, pr["means2d"], pr["cov2d"], fwd["point_list"], fwd["ranges"],
                         fwd["final_T"], fwd["n_contrib"], grad_field)
    gc, gq, gs = geom_backward(g, cam, rb["means2d"].astype(np.float32),
                               rb["cov2d"].astype(np.float32))
    return dict(cam=gc, z=np.zeros(g.n, np.float32), quats=gq, scales=gs,
                colours=rb["colours"].astype(np.float32), phase=rb["phase"].astype(np.float32),
                opac=rb["opac"].astype(np.float32), plane=rb["plane"].astype(np.float32),
                render=rb)


# ------------------------------------------------------------------ ASM ---

def fftfreq_f32(n: int, d: float) -> np.ndarray:
    """torch.fft.fftfreq(n, d) in float32: float32(bin) * float32(1/(n*d))."""
    k = np.fft.fftfreq(n, d=1.0 / n)
    return (k.astype(np.float32) * np.float32(1.0 / (n * d))).astype(np.float32)


def freq_grids(M: int, pitch: float):
    """FX, FY = meshgrid(fftshift(fftfreq)), indexing='ij' (python_function.py:137-142)."""
    f = np.fft.fftshift(fftfreq_f32(M, pitch))
    FX, FY = np.meshgrid(f, f, indexing="ij")
    return np.ascontiguousarray(FX, np.float32), np.ascontiguousarray(FY, np.float32)


def asm_spectral(re, im, FX, FY, wavelength, distance, aperture, pitch, adjoint=False):
    L = lib()
    nx, ny = re.shape
    ore = np.zeros_like(_f32(re))
    oim = np.zeros_like(_f32(im))
    L.oracle_asm_spectral(_f32(re), _f32(im), _f32(FX), _f32(FY), ore, oim, nx, ny,
                          np.float32(wavelength), np.float32(distance), np.float32(aperture),
                          np.float32(pitch), 1 if adjoint else 0)
    return ore, oim


def asm_consts(wavelength, distance, pitch, n):
    out = np.zeros(4, np.float32)
    lib().oracle_asm_consts(np.float32(wavelength), np.float32(distance), np.float32(pitch), n, out)
    return out


def zero_pad(field, size):
    """Centred zero pad, start = size//2 - n//2 (odak zero_pad, 'center')."""
    H, W = field.shape[-2:]
    out = np.zeros(field.shape[:-2] + tuple(size), dtype=np.complex128)
    r0, c0 = size[0] // 2 - H // 2, size[1] // 2 - W // 2
    out[..., r0:r0 + H, c0:c0 + W] = field
    return out


def crop_center(field, size):
    """Centred crop, start = M//2 - s//2 (odak crop_center with size)."""
    M0, M1 = field.shape[-2:]
    r0, c0 = M0 // 2 - size[0] // 2, M1 // 2 - size[1] // 2
    return field[..., r0:r0 + size[0], c0:c0 + size[1]]


def asm_forward(field, wavelength, pitch, distance, S, aperture):
    """BandlimitedPropagationFunction.forward (python_function.py:111-163)."""
    M = 2 * S
    padded = zero_pad(field, (M, M))
    ff = np.fft.fftshift(np.fft.fft2(padded))
    FX, FY = freq_grids(M, pitch)
    ore, oim = asm_spectral(ff.real, ff.imag, FX, FY, wavelength, distance, aperture, pitch)
    out = np.fft.ifft2(np.fft.ifftshift(ore.astype(np.float64) + 1j * oim.astype(np.float64)))
    return crop_center(out, (S, S))


def asm_adjoint(grad, H, W, wavelength, pitch, distance, S, aperture):
    """BandlimitedPropagationFunction.backward (python_function.py:166-218)."""
    M = 2 * S
    padded = zero_pad(grad, (M, M))
    gf = np.fft.fftshift(np.fft.fft2(padded))
    FX, FY = freq_grids(M, pitch)
    ore, oim = asm_spectral(gf.real, gf.imag, FX, FY, wavelength, distance, aperture, pitch,
                            adjoint=True)
    out = np.fft.ifft2(np.fft.ifftshift(ore.astype(np.float64) + 1j * oim.astype(np.float64)))
    return crop_center(out, (H, W))


def multiplane_forward(fields, wavelengths, distances, pitch, S, aperture):
    """Scene.splat's per-(p,c) loop and Python sum (model.py:1251-1272)."""
    P, C = fields.shape[:2]
    holo = np.zeros((C, S, S), np.complex128)
    for p in range(P):
        for c in range(C):
            holo[c] += asm_forward(fields[p, c], wavelengths[c], pitch, distances[p], S, aperture)
    return holo


def multiplane_adjoint(grad_holo, H, W, wavelengths, distances, pitch, S, aperture):
    C = grad_holo.shape[0]
    P = len(distances)
    out = np.zeros((P, C, H, W), np.complex128)
    for p in range(P):
        for c in range(C):
            out[p, c] = asm_adjoint(grad_holo[c], H, W, wavelengths[c], pitch, distances[p], S,
                                    aperture)
    return out


# ------------------------------------------------------- render preprocess ---
# Scene.render's glue ahead of splat_tile_cuda (model.py:1365-1402, 1105-1125,
# 594-608, 41-56; the world-to-view transform of Scene.splat, model.py:
# 1161-1162), restated in numpy float32 with one rounding per operation.

TWO_PI_F32 = np.float32(2.0 * np.pi)  # torch casts the Python scalar to float32


def _camera_points(means, R, T):
    """X @ R + T, left to right per component (model.py:1110)."""
    m = _f32(means)
    R = _f32(R).reshape(3, 3)
    T = _f32(T).reshape(3)
    out = np.empty_like(m)
    for j in range(3):
        out[:, j] = ((m[:, 0] * R[0, j] + m[:, 1] * R[1, j]) + m[:, 2] * R[2, j]) + T[j]
    return out


def _remainder_2pi(x):
    """torch.remainder(x, 2*pi) in float32: exact fmod, then the divisor's sign
    (model.py:602)."""
    x = _f32(x)
    r = np.fmod(x, TWO_PI_F32)
    fix = (r != 0) & ((r < 0) != (TWO_PI_F32 < 0))
    return np.where(fix, (r + TWO_PI_F32).astype(np.float32), r).astype(np.float32)


def _normalize(q):
    """F.normalize(q, dim=1): q / max(||q||_2, 1e-12)."""
    q = _f32(q)
    s = ((q[:, 0] * q[:, 0] + q[:, 1] * q[:, 1]) + q[:, 2] * q[:, 2]) + q[:, 3] * q[:, 3]
    nrm = np.maximum(np.sqrt(s), np.float32(1e-12)).astype(np.float32)
    return (q / nrm[:, None]).astype(np.float32), np.sqrt(s).astype(np.float32)


def _sigmoid(x):
    x = _f32(x)
    return (np.float32(1.0) / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def _one_hot_argmax(logits):
    """one_hot(argmax(., dim=1)): first maximal entry; NaN counts as maximal."""
    x = _f32(logits)
    n, P = x.shape
    best = np.zeros(n, np.int64)
    bv = x[:, 0].copy()
    for p in range(1, P):
        v = x[:, p]
        take = ~np.isnan(bv) & ((v > bv) | np.isnan(v))
        best = np.where(take, p, best)
        bv = np.where(take, v, bv)
    out = np.zeros((n, P), np.float32)
    out[np.arange(n), best] = 1.0
    return out


def _ste_softmax(logits):
    """softmax(logits / 0.001, dim=1) in float32 (STEFunction.backward)."""
    v = (_f32(logits) / np.float32(0.001)).astype(np.float32)
    e = np.exp(v - v.max(axis=1, keepdims=True)).astype(np.float32)
    return (e / e.sum(axis=1, dtype=np.float32, keepdims=True)).astype(np.float32)


def preprocess_select(means, R, T, near, far):
    """Selected parameter rows in ascending depth order (stable: equal depths
    keep the row order)."""
    cam = _camera_points(means, R, T)
    z = cam[:, 2]
    keep = np.nonzero((z > np.float32(near)) & (z < np.float32(far)) & (z >= 0))[0]
    order = np.argsort(z[keep], kind="stable")
    return keep[order].astype(np.int64)


def preprocess_forward(means, pre_quats, pre_scales, colours, pre_phase, pre_opac, pre_plane,
                       R, T, near=1.0, far=1000.0):
    """-> dict(cam, z, quats, scales, colours, phase, opacities, plane_probs, idxs)."""
    idx = preprocess_select(means, R, T, near, far)
    cam = _camera_points(_f32(means)[idx], R, T)
    q, _ = _normalize(_f32(pre_quats)[idx])
    return dict(cam=cam, z=cam[:, 2].copy(), quats=q,
                scales=np.exp(_f32(pre_scales)[idx]).astype(np.float32),
                colours=_f32(colours)[idx].copy(), phase=_remainder_2pi(_f32(pre_phase)[idx]),
                opacities=_sigmoid(_f32(pre_opac).reshape(-1)[idx]),
                plane_probs=_one_hot_argmax(_f32(pre_plane)[idx]), idxs=idx)


def preprocess_backward(grads, means, pre_quats, pre_scales, colours, pre_phase, pre_opac,
                        pre_plane, R, idxs):
    """grads: dict with keys cam, z (optional), quats, scales, colours, phase,
    opacities, plane_probs (selected rows) -> parameter gradients (N rows)."""
    n = _f32(means).shape[0]
    C = _f32(colours).shape[1]
    P = _f32(pre_plane).shape[1]
    R = _f32(R).reshape(3, 3)
    idx = np.asarray(idxs, np.int64)
    out = dict(means=np.zeros((n, 3), np.float32), pre_quats=np.zeros((n, 4), np.float32),
               pre_scales=np.zeros((n, 3), np.float32), colours=np.zeros((n, C), np.float32),
               pre_phase=np.zeros((n, C), np.float32), pre_opac=np.zeros(n, np.float32),
               pre_plane=np.zeros((n, P), np.float32))
    gc = _f32(grads["cam"]).copy()
    if grads.get("z") is not None:
        gc[:, 2] = gc[:, 2] + _f32(grads["z"])
    for k in range(3):
        out["means"][idx, k] = (gc[:, 0] * R[k, 0] + gc[:, 1] * R[k, 1]) + gc[:, 2] * R[k, 2]
    q = _f32(pre_quats)[idx]
    y, raw = _normalize(q)
    gq = _f32(grads["quats"])
    dot = ((y[:, 0] * gq[:, 0] + y[:, 1] * gq[:, 1]) + y[:, 2] * gq[:, 2]) + y[:, 3] * gq[:, 3]
    big = raw > np.float32(1e-12)
    safe = np.where(big, raw, np.float32(1.0)).astype(np.float32)
    dq = np.where(big[:, None], (gq - y * dot[:, None]) / safe[:, None], gq / np.float32(1e-12))
    out["pre_quats"][idx] = dq.astype(np.float32)
    out["pre_scales"][idx] = _f32(grads["scales"]) * np.exp(_f32(pre_scales)[idx])
    out["colours"][idx] = _f32(grads["colours"])
    out["pre_phase"][idx] = _f32(grads["phase"])
    s = _sigmoid(_f32(pre_opac).reshape(-1)[idx])
    out["pre_opac"][idx] = _f32(grads["opacities"]) * (s * (np.float32(1.0) - s))
    out["pre_plane"][idx] = _f32(grads["plane_probs"]) * _ste_softmax(_f32(pre_plane)[idx])
    return out


# ----------------------------------------------------- optimizer step
# train.py:319-324: torch.nn.utils.clip_grad_norm_(parameters, 1.0), then
# Adan.step() (utils/optimizer.py:288-466), whose foreach path
# _multi_tensor_adan (:538-589) the reference runs.  numpy float32, op by op.

def clip_grad_norm(grads, max_norm):
    """(total_norm, clip_coef, scaled grads): total = ||all grads||_2
    (accumulated in float64, rounded once), coef = clamp(max_norm / (total +
    1e-6), max=1) in float32 with NaN propagating (torch.clamp), every
    gradient times coef (torch/nn/utils/clip_grad.py)."""
    gs = [_f32(g) for g in grads]
    ss = sum(float(np.sum(g.astype(np.float64) ** 2)) for g in gs)
    total = np.float32(np.sqrt(ss))
    coef = np.float32(max_norm) / (total + np.float32(1e-6))
    coef = np.float32(1.0) if coef > np.float32(1.0) else np.float32(coef)
    return total, coef, [g * coef for g in gs]


def adan_step(p, g, exp_avg, exp_avg_sq, exp_avg_diff, neg_pre_grad, *, lr, step,
              betas=(0.98, 0.92, 0.99), eps=1e-8, weight_decay=0.0, no_prox=False,
              clip=1.0, init_neg_pre_grad=None):
    """One Adan update of one tensor (optimizer.py:429-441 state set-up,
    :556-589 the update); returns the new (p, g, exp_avg, exp_avg_sq,
    exp_avg_diff, neg_pre_grad).  Python-float scalars (bias corrections,
    step sizes) are formed in double and rounded to float32 where they meet
    the tensors, as torch does; init_neg_pre_grad defaults to step == 1."""
    f = np.float32
    b1, b2, b3 = (float(b) for b in betas)
    p, g, m, n, d = (_f32(x).copy() for x in (p, g, exp_avg, exp_avg_sq, exp_avg_diff))
    q = _f32(neg_pre_grad).copy()
    if init_neg_pre_grad is None:
        init_neg_pre_grad = step == 1
    if init_neg_pre_grad:
        q = g * f(-clip)                                 # p.grad.clone().mul_(-clip)
    bc1, bc2, bc3 = 1.0 - b1 ** step, 1.0 - b2 ** step, 1.0 - b3 ** step
    g = g * f(clip)
    q = q + g
    m = m * f(b1)
    m = m + f(1.0 - b1) * g
    d = d * f(b2)
    d = d + f(1.0 - b2) * q
    q = q * f(b2)
    q = q + g
    n = n * f(b3)
    n = n + f(1.0 - b3) * q * q
    denom = np.sqrt(n)
    denom = denom / f(np.sqrt(bc3))
    denom = denom + f(eps)
    step_size_diff = f(lr * b2 / bc2)
    step_size = f(lr / bc1)
    if no_prox:
        p = p * f(1.0 - lr * weight_decay)
        p = p + (-step_size) * (m / denom)
        p = p + (-step_size_diff) * (d / denom)
    else:
        p = p + (-step_size) * (m / denom)
        p = p + (-step_size_diff) * (d / denom)
        p = p / f(1.0 + lr * weight_decay)
    q = np.zeros_like(q) + f(-1.0) * g
    return p, g, m, n, d, q


# ------------------------------------------------- loss-side reconstruction
# propagator._reconstruct_impl (utils/propagator.py:548-636) with the
# reference's own band-limited ASM (asm_forward above) as the propagation:
# float64 fields w a e^{i s phi}, propagated to each depth, |u|^2.

def reconstruct(phases, amplitude, wavelengths, pitch, distances, S, aperture, powers,
                scales=None, get_complex=False):
    """-> (F, D, C, S, S) intensities (complex with get_complex)."""
    phases = np.asarray(phases, np.float64)
    amplitude = np.asarray(amplitude, np.float64)
    F, C, D = phases.shape[0], amplitude.shape[0], len(distances)
    powers = np.asarray(powers, np.float64).reshape(F, C)
    scales = np.ones(C) if scales is None else np.asarray(scales, np.float64)
    out = np.zeros((F, D, C, S, S), np.complex128 if get_complex else np.float64)
    for f in range(F):
        for c in range(C):
            if powers[f, c] == 0:
                continue
            field = powers[f, c] * amplitude[c] * np.exp(1j * phases[f] * scales[c])
            for d in range(D):
                u = asm_forward(field, wavelengths[c], pitch, distances[d], S, aperture)
                out[f, d, c] = u if get_complex else np.abs(u) ** 2
    return out


def reconstruct_backward(grad, phases, amplitude, wavelengths, pitch, distances, S, aperture,
                         powers, scales=None):
    """Gradients of sum(grad * reconstruct(...)) w.r.t. (phases, amplitude):
    dL/du = 2 g u, the propagation's adjoint (asm_adjoint), then
    dL/da = w Re(gz e^{-i s phi}), dL/dphi = s w a Im(gz e^{-i s phi})."""
    phases = np.asarray(phases, np.float64)
    amplitude = np.asarray(amplitude, np.float64)
    grad = np.asarray(grad, np.float64)
    F, C, D = phases.shape[0], amplitude.shape[0], len(distances)
    powers = np.asarray(powers, np.float64).reshape(F, C)
    scales = np.ones(C) if scales is None else np.asarray(scales, np.float64)
    g_ph = np.zeros_like(phases)
    g_amp = np.zeros_like(amplitude)
    for f in range(F):
        for c in range(C):
            w = powers[f, c]
            if w == 0:
                continue
            e = np.exp(1j * phases[f] * scales[c])
            field = w * amplitude[c] * e
            gz = np.zeros((S, S), np.complex128)
            for d in range(D):
                u = asm_forward(field, wavelengths[c], pitch, distances[d], S, aperture)
                gz += asm_adjoint(2.0 * grad[f, d, c] * u, S, S, wavelengths[c], pitch,
                                  distances[d], S, aperture)
            t = gz * np.conj(e)
            g_amp[c] += w * t.real
            g_ph[f] += scales[c] * w * amplitude[c] * t.imag
    return g_ph, g_amp


# ----------------------------------------------------------- SSIM (fast_ssim)
# Restates the reference's fused SSIM (cuda_prop/cov3d_cuda/conv.cu:935-1135)
# in float64: the 11x11 window as the outer product of the normalised 1-D
# Gaussian (sigma 1.5; the reference's 2-D constants G_000..G_120 are those
# products rounded to 1e-10), zero padding, the map's four factors and the
# image-1 gradient through the window statistics.

def ssim_window_1d() -> np.ndarray:
    k = np.arange(11, dtype=np.float64) - 5.0
    w = np.exp(-k * k / (2.0 * 1.5 * 1.5))
    return w / w.sum()


def _window_sum(a: np.ndarray) -> np.ndarray:
    """sum over the 11x11 window (weights w_i w_j) of a zero-padded (..., H, W)."""
    w = ssim_window_1d()
    H, W = a.shape[-2:]
    p = np.zeros(a.shape[:-2] + (H + 10, W + 10), dtype=np.float64)
    p[..., 5:5 + H, 5:5 + W] = a
    out = np.zeros(a.shape, dtype=np.float64)
    for i in range(11):
        for j in range(11):
            out += w[i] * w[j] * p[..., i:i + H, j:j + W]
    return out


def _ssim_terms(x, y, C1, C2):
    mu1, mu2 = _window_sum(x), _window_sum(y)
    s11 = _window_sum(x * x) - mu1 * mu1
    s22 = _window_sum(y * y) - mu2 * mu2
    s12 = _window_sum(x * y) - mu1 * mu2
    C = 2.0 * mu1 * mu2 + C1
    D = 2.0 * s12 + C2
    A = mu1 * mu1 + mu2 * mu2 + C1
    B = s11 + s22 + C2
    return mu1, mu2, A, B, C, D


def ssim_map(img1, img2, C1=0.01 ** 2, C2=0.03 ** 2) -> np.ndarray:
    """SSIM map (C, H, W) in float64 (conv.cu:993-1001)."""
    x = np.asarray(img1, dtype=np.float64)
    y = np.asarray(img2, dtype=np.float64)
    _, _, A, B, C, D = _ssim_terms(x, y, C1, C2)
    return (C * D) / (A * B)


def ssim_backward(img1, img2, grad_map, C1=0.01 ** 2, C2=0.03 ** 2) -> np.ndarray:
    """d(sum grad_map * map)/d img1 in float64 (conv.cu:1075-1130): the map's
    partials with respect to mu1, window(x^2) and window(xy), pulled back
    through the (symmetric) window."""
    x = np.asarray(img1, dtype=np.float64)
    y = np.asarray(img2, dtype=np.float64)
    g = np.asarray(grad_map, dtype=np.float64)
    mu1, mu2, A, B, C, D = _ssim_terms(x, y, C1, C2)
    AB = A * B
    d_mu1 = g * ((mu2 * 2.0 * D) / AB - (mu2 * 2.0 * C) / AB - (mu1 * 2.0 * C * D) / (A * A * B)
                 + (mu1 * 2.0 * C * D) / (AB * B))
    d_s11 = g * ((-C * D) / (AB * B))
    d_s12 = g * ((2.0 * C) / AB)
    return _window_sum(d_mu1) + 2.0 * x * _window_sum(d_s11) + y * _window_sum(d_s12)


# ----------------------------------------------------- sparse Adam (spadam.cu)

def sparse_adam_update(param, grad, exp_avg, exp_avg_sq, visible, lr, b1, b2, eps):
    """Restates sparse_adam_kernel (cuda_prop/cov3d_cuda/spadam.cu:8-36) in
    float32, op for op: returns updated copies of (param, exp_avg,
    exp_avg_sq).  param/exp_avg/exp_avg_sq (B, N, D), grad (B, V, D),
    visible (V) row indices; rows outside [0, N) are skipped."""
    p = np.array(param, dtype=np.float32, copy=True)
    m = np.array(exp_avg, dtype=np.float32, copy=True)
    s = np.array(exp_avg_sq, dtype=np.float32, copy=True)
    g = np.asarray(grad, dtype=np.float32)
    lr, b1, b2, eps = (np.float32(v) for v in (lr, b1, b2, eps))
    one = np.float32(1.0)
    N = p.shape[1]
    for v, row in enumerate(np.asarray(visible, dtype=np.int64)):
        if row < 0 or row >= N:
            continue
        gr = g[:, v, :]
        mm = b1 * m[:, row, :] + (one - b1) * gr
        ss = b2 * s[:, row, :] + (one - b2) * gr * gr
        step = (-lr * mm) / (np.sqrt(ss) + eps)
        p[:, row, :] = p[:, row, :] + step
        m[:, row, :] = mm
        s[:, row, :] = ss
    return p, m, s
