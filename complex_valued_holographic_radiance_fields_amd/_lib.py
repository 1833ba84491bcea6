"""ctypes binding of ``lib/libhrf.so`` (the C ABI declared in include/hrf.h).

torch is imported first so that the HIP runtime torch ships with is the one
the library binds to (both carry the soname ``libamdhip64.so.7``); torch is
used only for device memory and the current stream.  There is no fallback:
if the library is missing or fails to load, importing the package raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (loads the HIP runtime before libhrf.so)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libhrf.so")

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_sz = ctypes.c_size_t


class HrfGaussians(ctypes.Structure):
    _fields_ = [
        ("cam_means", _vp), ("z_vals", _vp), ("quats", _vp), ("scales", _vp),
        ("colours", _vp), ("phase", _vp), ("opacities", _vp), ("plane_probs", _vp),
        ("n", _i64), ("channels", _i32), ("planes", _i32),
    ]


class HrfCamera(ctypes.Structure):
    _fields_ = [
        ("fx", _f32), ("fy", _f32), ("px", _f32), ("py", _f32),
        ("view_matrix", _vp), ("width", _i32), ("height", _i32),
        ("near_plane", _f32), ("far_plane", _f32),
    ]


class HrfSceneParams(ctypes.Structure):
    _fields_ = [
        ("means", ctypes.c_void_p), ("pre_quats", ctypes.c_void_p),
        ("pre_scales", ctypes.c_void_p), ("colours", ctypes.c_void_p),
        ("pre_phase", ctypes.c_void_p), ("pre_opacities", ctypes.c_void_p),
        ("pre_plane", ctypes.c_void_p), ("n", ctypes.c_int64), ("channels", ctypes.c_int32),
        ("planes", ctypes.c_int32),
    ]


class HrfSelectedGrads(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in
                ("cam", "z", "quats", "scales", "colours", "phase", "opacities", "plane_probs")]


class HrfParamGrads(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in
                ("means", "pre_quats", "pre_scales", "colours", "pre_phase", "pre_opacities",
                 "pre_plane")]


class HrfAdanTensor(ctypes.Structure):
    _fields_ = [("param", _vp), ("grad", _vp), ("exp_avg", _vp), ("exp_avg_sq", _vp),
                ("exp_avg_diff", _vp), ("neg_pre_grad", _vp), ("numel", _i64), ("lr", _f64),
                ("step", _i64), ("init_neg_pre_grad", _i32)]


class HrfAdanConfig(ctypes.Structure):
    _fields_ = [("beta1", _f64), ("beta2", _f64), ("beta3", _f64), ("eps", _f64),
                ("weight_decay", _f64), ("clip_global_grad_norm", _f64), ("no_prox", _i32)]


_P = ctypes.POINTER
# name -> (restype, argtypes); exactly the entry points of include/hrf.h.
SIGNATURES = {
    "hrf_last_error": (ctypes.c_char_p, []),
    "hrf_version": (ctypes.c_char_p, []),
    "hrf_raster_geom_workspace_size": (_sz, [_i64, _i32, _i32]),
    "hrf_raster_binning_workspace_size": (_sz, [_i64, _i32, _i32]),
    "hrf_raster_forward_prepare": (ctypes.c_int, [
        _P(HrfGaussians), _P(HrfCamera), _vp, _sz, _vp, _P(_i64), _P(_i64)]),
    "hrf_raster_forward_render": (ctypes.c_int, [
        _P(HrfGaussians), _P(HrfCamera), _vp, _sz, _vp, _sz, _i64, _i64,
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "hrf_raster_plane_lists_size": (_sz, [_i64, _i32, _i32, _i32]),
    "hrf_raster_backward_workspace_size": (_sz, [_i64, _i32, _i32]),
    "hrf_raster_backward_prepare": (ctypes.c_int, [
        _P(HrfGaussians), _P(HrfCamera), _i64, _vp, _sz, _vp, _sz, _vp]),
    "hrf_raster_backward": (ctypes.c_int, [
        _P(HrfGaussians), _P(HrfCamera), _vp, _vp, _vp, _vp, _vp, _i64, _vp, _sz, _vp, _sz,
        _vp, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hrf_asm_multidistance_workspace_size": (_sz, [_i32, _i32]),
    "hrf_asm_multidistance_forward": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32, _i32, _vp,
                                                     _vp, _f64, _f32, _vp, _vp, _sz, _vp]),
    "hrf_asm_multidistance_adjoint": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32, _i32, _vp,
                                                     _vp, _f64, _f32, _vp, _vp, _sz, _vp]),
    "hrf_recon_fields": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _i32,
                                        _vp, _vp]),
    "hrf_recon_intensity": (ctypes.c_int, [_vp, _i64, _vp, _vp]),
    "hrf_recon_intensity_backward": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp]),
    "hrf_recon_fields_backward": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i64, _vp, _vp, _vp, _vp,
                                                 _i32, _vp, _vp, _vp, _vp]),
    "hrf_grad_norm_workspace_size": (_sz, [_P(_i64), _i32]),
    "hrf_grad_norm": (ctypes.c_int, [_P(_vp), _P(_i64), _i32, _f32, _vp, _vp, _vp, _sz, _vp]),
    "hrf_scale_grads": (ctypes.c_int, [_P(_vp), _P(_i64), _i32, _vp, _vp]),
    "hrf_adan_step": (ctypes.c_int, [_P(HrfAdanTensor), _i32, _P(HrfAdanConfig), _vp, _vp]),
    "hrf_grad_norm_static": (ctypes.c_int, [_P(_vp), _P(_i64), _i32, _f32, _vp, _vp, _vp]),
    "hrf_ssim_map": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, _f32, _f32, _vp, _vp]),
    "hrf_ssim_backward": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _f32, _f32, _vp, _vp]),
    "hrf_sparse_adam_update": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                              _f32, _f32, _f32, _f32, _vp]),
    "hrf_preprocess_workspace_size": (_sz, [_i64, _i32, _i32]),
    "hrf_preprocess_select": (ctypes.c_int, [_P(HrfSceneParams), _vp, _vp, _f32, _f32, _vp, _sz,
                                             _vp, _P(_i64)]),
    "hrf_preprocess_forward": (ctypes.c_int, [_P(HrfSceneParams), _vp, _vp, _vp, _sz, _i64,
                                              _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hrf_preprocess_backward": (ctypes.c_int, [_P(HrfSceneParams), _vp, _vp, _i64,
                                               _P(HrfSelectedGrads), _P(HrfParamGrads), _vp,
                                               _sz, _vp]),
    "hrf_cov3d_forward": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp]),
    "hrf_cov3d_backward": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp, _vp, _vp]),
    "hrf_jacobian_forward": (ctypes.c_int, [_vp, _i64, _f32, _f32, _i32, _i32, _f32, _f32,
                                            _vp, _vp]),
    "hrf_jacobian_backward": (ctypes.c_int, [_vp, _vp, _i64, _f32, _f32, _i32, _i32, _f32,
                                             _f32, _vp, _vp]),
    "hrf_cov2d_forward": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _f32, _f32, _i32, _i32,
                                         _f32, _f32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hrf_cov2d_backward": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                                          _f32, _f32, _i32, _i32, _f32, _f32, _vp, _vp, _vp,
                                          _vp]),
    "hrf_means2d_forward": (ctypes.c_int, [_vp, _i64, _f32, _f32, _f32, _f32, _f32, _f32, _vp,
                                           _vp]),
    "hrf_means2d_backward": (ctypes.c_int, [_vp, _vp, _i64, _f32, _f32, _f32, _f32, _f32, _f32,
                                            _vp, _vp]),
    "hrf_invert_cov2d_forward": (ctypes.c_int, [_vp, _i64, _vp, _vp]),
    "hrf_invert_cov2d_backward": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp]),
    "hrf_asm_spectral_forward": (ctypes.c_int, [
        _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _f32, _f32, _f32, _vp]),
    "hrf_asm_spectral_backward": (ctypes.c_int, [
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _f32, _f32, _f32, _vp]),
    "hrf_asm_workspace_size": (_sz, [_i32, _i32, _i32]),
    "hrf_asm_forward": (ctypes.c_int, [
        _vp, _i32, _i32, _i32, _f32, _f64, _f32, _f32, _vp, _vp, _sz, _vp]),
    "hrf_asm_adjoint": (ctypes.c_int, [
        _vp, _i32, _i32, _i32, _f32, _f64, _f32, _f32, _vp, _vp, _sz, _vp]),
    "hrf_asm_multiplane_forward": (ctypes.c_int, [
        _vp, _i32, _i32, _i32, _i32, _i32, _P(_f32), _P(_f32), _f64, _f32, _vp, _vp, _sz,
        _vp]),
    "hrf_asm_multiplane_adjoint": (ctypes.c_int, [
        _vp, _i32, _i32, _i32, _i32, _i32, _P(_f32), _P(_f32), _f64, _f32, _vp, _vp, _sz,
        _vp]),
    "hrf_release_caches": (None, []),
    "hrf_trace_enable": (ctypes.c_int, [ctypes.c_int]),
    "hrf_trace_only": (ctypes.c_int, [ctypes.c_char_p]),
    "hrf_trace_reset": (None, []),
    "hrf_trace_read": (ctypes.c_int, [ctypes.c_char_p, _P(_i64), _P(_f64)]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libhrf.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build the gfx950 HIP library first "
            "(python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status: int) -> None:
    if status != 0:
        msg = load().hrf_last_error()
        raise RuntimeError((msg or b"hrf: unknown error").decode(errors="replace"))


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def trace_enable(on: bool) -> None:
    check(load().hrf_trace_enable(1 if on else 0))


def trace_only(stage: str | None) -> None:
    """Trace only `stage` (None: every stage)."""
    check(load().hrf_trace_only(stage.encode() if stage else None))


def trace_reset() -> None:
    load().hrf_trace_reset()


def trace_read(stage: str):
    """(launches, total milliseconds) of a traced stage since the last reset."""
    n = _i64(0)
    ms = _f64(0.0)
    check(load().hrf_trace_read(stage.encode(), ctypes.byref(n), ctypes.byref(ms)))
    return int(n.value), float(ms.value)


# Grow-only scratch buffers, one per (purpose, device, stream, host thread).
# A workspace is only touched by the kernels of the call that receives it, all
# enqueued on that call's stream, so handing the same memory to the next call
# from the same thread on the same stream is ordered by the stream itself
# (another thread could enqueue between a call's two phases, hence the thread
# in the key).
_WORKSPACES: dict = {}


def workspace(purpose: str, device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """A uint8 device buffer of at least `nbytes` bytes for `purpose` on
    (`device`, `stream`) for the calling host thread."""
    key = (purpose, str(device), int(stream), threading.get_ident())
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = buf
    return buf


def release_workspaces() -> None:
    """Drops the cached workspaces (the memory returns to torch's allocator)."""
    _WORKSPACES.clear()

