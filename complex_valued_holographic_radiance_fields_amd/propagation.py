"""Host side of the band-limited ASM propagator (C ABI calls on torch memory).

``propagate`` / ``propagate_adjoint`` are BandlimitedPropagationFunction's
forward/backward (cuda_prop/python_function.py:111-218); ``multiplane`` /
``multiplane_adjoint`` fuse Scene.splat's per-(plane, wavelength) loop and
Python sum (model.py:1251-1272); ``multidistance`` / ``multidistance_adjoint``
propagate one field per wavelength to many distances with the forward
transforms shared; ``spectral_forward`` / ``spectral_backward``
are the ``cuda_modules.bandlimited_propagation_forward/backward`` bindings
(cuda_prop/cpp/module_def.cpp:4-24).
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _lib


def _as_float(x) -> float:
    if isinstance(x, torch.Tensor):
        return float(x.detach().reshape(-1)[0].item())
    return float(x)


def _square_size(size) -> int:
    if isinstance(size, int):
        return int(size)
    s = [int(v) for v in size]
    if len(s) != 2 or s[0] != s[1]:
        raise RuntimeError(f"propagation size must be square (S, S); got {s} "
                           "(the reference kernel indexes non-square grids incorrectly)")
    return s[0]


def _c64(t: torch.Tensor, name: str) -> torch.Tensor:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (the HIP propagator has no CPU path)")
    if t.dtype != torch.complex64:
        t = t.to(torch.complex64)
    return t.contiguous()


def _workspace(P: int, C: int, S: int, dev) -> tuple[torch.Tensor, int]:
    nbytes = _lib.load().hrf_asm_workspace_size(P, C, S)
    return _lib.workspace("asm", dev, _lib.stream_ptr(dev), nbytes), nbytes


def propagate(field: torch.Tensor, wavelength, pixel_pitch, distance, size,
              aperture_size=-1.0) -> torch.Tensor:
    """(H,W) complex field -> (S,S) complex field at ``distance``."""
    field = _c64(field, "field")
    if field.dim() != 2:
        raise RuntimeError(f"field must be 2-D (H, W); got {tuple(field.shape)}")
    S = _square_size(size)
    H, W = field.shape
    out = torch.empty((S, S), dtype=torch.complex64, device=field.device)
    lib = _lib.load()
    with torch.cuda.device(field.device):
        ws, nb = _workspace(1, 1, S, field.device)
        _lib.check(lib.hrf_asm_forward(field.data_ptr(), H, W, S, _as_float(wavelength),
                                       _as_float(pixel_pitch), _as_float(distance),
                                       _as_float(aperture_size), out.data_ptr(), ws.data_ptr(),
                                       nb, _lib.stream_ptr(field.device)))
    return out


def propagate_adjoint(grad_out: torch.Tensor, input_size, wavelength, pixel_pitch, distance,
                      size, aperture_size=-1.0) -> torch.Tensor:
    """(S,S) gradient -> (H,W) gradient (exact adjoint of ``propagate``)."""
    grad_out = _c64(grad_out, "grad_output")
    S = _square_size(size)
    if tuple(grad_out.shape) != (S, S):
        raise RuntimeError(f"grad_output must have shape {(S, S)}, got {tuple(grad_out.shape)}")
    H, W = int(input_size[0]), int(input_size[1])
    out = torch.empty((H, W), dtype=torch.complex64, device=grad_out.device)
    lib = _lib.load()
    with torch.cuda.device(grad_out.device):
        ws, nb = _workspace(1, 1, S, grad_out.device)
        _lib.check(lib.hrf_asm_adjoint(grad_out.data_ptr(), H, W, S, _as_float(wavelength),
                                       _as_float(pixel_pitch), _as_float(distance),
                                       _as_float(aperture_size), out.data_ptr(), ws.data_ptr(),
                                       nb, _lib.stream_ptr(grad_out.device)))
    return out


def _host_f32(vals: Sequence[float]):
    arr = (ctypes.c_float * len(vals))(*[_as_float(v) for v in vals])
    return arr


def multiplane(fields: torch.Tensor, wavelengths, pixel_pitch, distances, size,
               aperture_size=-1.0) -> torch.Tensor:
    """fields (P,C,H,W) -> hologram (C,S,S) = sum_p propagate(fields[p,c],
    wavelengths[c], distances[p])."""
    fields = _c64(fields, "fields")
    if fields.dim() != 4:
        raise RuntimeError(f"fields must be (P, C, H, W); got {tuple(fields.shape)}")
    P, C, H, W = fields.shape
    wl = [_as_float(w) for w in (wavelengths.tolist() if isinstance(wavelengths, torch.Tensor)
                                 else wavelengths)]
    ds = [_as_float(d) for d in (distances.tolist() if isinstance(distances, torch.Tensor)
                                 else distances)]
    if len(wl) != C or len(ds) != P:
        raise RuntimeError(f"need {C} wavelengths and {P} distances (got {len(wl)}, {len(ds)})")
    S = _square_size(size)
    out = torch.empty((C, S, S), dtype=torch.complex64, device=fields.device)
    lib = _lib.load()
    with torch.cuda.device(fields.device):
        ws, nb = _workspace(P, C, S, fields.device)
        _lib.check(lib.hrf_asm_multiplane_forward(
            fields.data_ptr(), P, C, H, W, S, _host_f32(wl), _host_f32(ds),
            _as_float(pixel_pitch), _as_float(aperture_size), out.data_ptr(), ws.data_ptr(), nb,
            _lib.stream_ptr(fields.device)))
    return out


def multiplane_adjoint(grad_holo: torch.Tensor, field_hw, wavelengths, pixel_pitch, distances,
                       size, aperture_size=-1.0) -> torch.Tensor:
    grad_holo = _c64(grad_holo, "grad_hologram")
    C = grad_holo.shape[0]
    wl = [_as_float(w) for w in (wavelengths.tolist() if isinstance(wavelengths, torch.Tensor)
                                 else wavelengths)]
    ds = [_as_float(d) for d in (distances.tolist() if isinstance(distances, torch.Tensor)
                                 else distances)]
    P = len(ds)
    S = _square_size(size)
    H, W = int(field_hw[0]), int(field_hw[1])
    if tuple(grad_holo.shape) != (C, S, S) or len(wl) != C:
        raise RuntimeError(f"grad_hologram must be (C,S,S)=({len(wl)},{S},{S}); "
                           f"got {tuple(grad_holo.shape)}")
    out = torch.empty((P, C, H, W), dtype=torch.complex64, device=grad_holo.device)
    lib = _lib.load()
    with torch.cuda.device(grad_holo.device):
        ws, nb = _workspace(P, C, S, grad_holo.device)
        _lib.check(lib.hrf_asm_multiplane_adjoint(
            grad_holo.data_ptr(), P, C, H, W, S, _host_f32(wl), _host_f32(ds),
            _as_float(pixel_pitch), _as_float(aperture_size), out.data_ptr(), ws.data_ptr(), nb,
            _lib.stream_ptr(grad_holo.device)))
    return out


def _floats(vals):
    return [_as_float(v) for v in (vals.tolist() if isinstance(vals, torch.Tensor) else vals)]


def multidistance(fields: torch.Tensor, wavelengths, pixel_pitch, distances, size,
                  aperture_size=-1.0) -> torch.Tensor:
    """fields (C,H,W) -> (D,C,S,S) with out[d,c] = propagate(fields[c],
    wavelengths[c], distances[d]); each channel is transformed once for all
    distances (the propagation microbench runs BandlimitedPropagation per
    (distance, wavelength), python_function.py:220-226)."""
    fields = _c64(fields, "fields")
    if fields.dim() != 3:
        raise RuntimeError(f"fields must be (C, H, W); got {tuple(fields.shape)}")
    C, H, W = fields.shape
    wl, ds = _floats(wavelengths), _floats(distances)
    if len(wl) != C or len(ds) < 1:
        raise RuntimeError(f"need {C} wavelengths and at least one distance")
    S = _square_size(size)
    out = torch.empty((len(ds), C, S, S), dtype=torch.complex64, device=fields.device)
    lib = _lib.load()
    with torch.cuda.device(fields.device):
        nb = lib.hrf_asm_multidistance_workspace_size(C, S)
        ws = _lib.workspace("asm_md", fields.device, _lib.stream_ptr(fields.device), nb)
        _lib.check(lib.hrf_asm_multidistance_forward(
            fields.data_ptr(), len(ds), C, H, W, S, _host_f32(wl), _host_f32(ds),
            _as_float(pixel_pitch), _as_float(aperture_size), out.data_ptr(), ws.data_ptr(), nb,
            _lib.stream_ptr(fields.device)))
    return out


def multidistance_adjoint(grad_out: torch.Tensor, field_hw, wavelengths, pixel_pitch,
                          distances, size, aperture_size=-1.0) -> torch.Tensor:
    """(D,C,S,S) gradient -> (C,H,W) gradient (exact adjoint of
    ``multidistance``)."""
    grad_out = _c64(grad_out, "grad_output")
    wl, ds = _floats(wavelengths), _floats(distances)
    C, D = len(wl), len(ds)
    S = _square_size(size)
    H, W = int(field_hw[0]), int(field_hw[1])
    if tuple(grad_out.shape) != (D, C, S, S):
        raise RuntimeError(f"grad_output must be (D,C,S,S)=({D},{C},{S},{S}); "
                           f"got {tuple(grad_out.shape)}")
    out = torch.empty((C, H, W), dtype=torch.complex64, device=grad_out.device)
    lib = _lib.load()
    with torch.cuda.device(grad_out.device):
        nb = lib.hrf_asm_multidistance_workspace_size(C, S)
        ws = _lib.workspace("asm_md", grad_out.device, _lib.stream_ptr(grad_out.device), nb)
        _lib.check(lib.hrf_asm_multidistance_adjoint(
            grad_out.data_ptr(), D, C, H, W, S, _host_f32(wl), _host_f32(ds),
            _as_float(pixel_pitch), _as_float(aperture_size), out.data_ptr(), ws.data_ptr(), nb,
            _lib.stream_ptr(grad_out.device)))
    return out


class MultiDistancePropagation(torch.autograd.Function):
    """Differentiable ``multidistance``."""

    @staticmethod
    def forward(ctx, fields, wavelengths, pixel_pitch, distances, size, aperture_size=-1.0):
        ctx.args = (tuple(fields.shape[1:]), wavelengths, pixel_pitch, distances, size,
                    aperture_size)
        return multidistance(fields, wavelengths, pixel_pitch, distances, size, aperture_size)

    @staticmethod
    def backward(ctx, grad_out):
        hw, wl, pitch, ds, size, ap = ctx.args
        return (multidistance_adjoint(grad_out, hw, wl, pitch, ds, size, ap), None, None, None,
                None, None)


def _spectral(args, adjoint: bool):
    if adjoint:
        g_re, g_im, f_re, f_im, FX, FY, wavelength, distance, aperture, pitch = args
        re, im = g_re, g_im
    else:
        re, im, FX, FY, wavelength, distance, aperture, pitch = args
    ts = [t.contiguous() for t in (re, im, FX, FY)]
    for t in ts:
        if not t.is_cuda or t.dtype != torch.float32:
            raise RuntimeError("spectral inputs must be float32 GPU tensors")
        if t.shape != ts[0].shape or t.dim() != 2:
            raise RuntimeError("spectral inputs must share one 2-D shape")
    nx, ny = ts[0].shape
    out_re = torch.zeros_like(ts[0])
    out_im = torch.zeros_like(ts[0])
    lib = _lib.load()
    with torch.cuda.device(ts[0].device):
        s = _lib.stream_ptr(ts[0].device)
        if adjoint:
            fr = f_re.contiguous()
            fi = f_im.contiguous()
            _lib.check(lib.hrf_asm_spectral_backward(
                ts[0].data_ptr(), ts[1].data_ptr(), fr.data_ptr(), fi.data_ptr(),
                ts[2].data_ptr(), ts[3].data_ptr(), out_re.data_ptr(), out_im.data_ptr(), nx, ny,
                _as_float(wavelength), _as_float(distance), _as_float(aperture),
                _as_float(pitch), s))
        else:
            _lib.check(lib.hrf_asm_spectral_forward(
                ts[0].data_ptr(), ts[1].data_ptr(), ts[2].data_ptr(), ts[3].data_ptr(),
                out_re.data_ptr(), out_im.data_ptr(), nx, ny, _as_float(wavelength),
                _as_float(distance), _as_float(aperture), _as_float(pitch), s))
    return [out_re, out_im]


def spectral_forward(re, im, FX, FY, wavelength, distance, aperture_size, pixel_pitch):
    """cuda_modules.bandlimited_propagation_forward -> [re, im]."""
    return _spectral((re, im, FX, FY, wavelength, distance, aperture_size, pixel_pitch), False)


def spectral_backward(grad_re, grad_im, field_re, field_im, FX, FY, wavelength, distance,
                      aperture_size, pixel_pitch):
    """cuda_modules.bandlimited_propagation_backward -> [re, im]."""
    return _spectral((grad_re, grad_im, field_re, field_im, FX, FY, wavelength, distance,
                      aperture_size, pixel_pitch), True)
