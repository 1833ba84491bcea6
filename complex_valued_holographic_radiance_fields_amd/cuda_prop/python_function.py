"""Drop-in for ``cuda_prop/python_function.py`` of the reference.

``BandlimitedPropagationFunction`` / ``BandlimitedPropagation`` keep the
reference signatures (python_function.py:109-226); ``cuda_module`` exposes
the ``cuda_modules`` spectral bindings (cpp/module_def.cpp:53-58).  The
computation runs in the gfx950 HIP library; there is no CPU path.
"""
from __future__ import annotations

import types
from typing import Tuple

import torch
from torch.autograd import Function

from .. import propagation as _prop

cuda_module = types.SimpleNamespace(
    bandlimited_propagation_forward=_prop.spectral_forward,
    bandlimited_propagation_backward=_prop.spectral_backward,
)


def calculate_padding(original_size: int, target_size: int) -> Tuple[int, int]:
    """Left/right padding split (python_function.py:29-33)."""
    pad_size = target_size - original_size
    pad_left = pad_size // 2
    return pad_left, pad_size - pad_left


class BandlimitedPropagationFunction(Function):
    """Band-limited ASM propagation of one (H,W) complex field to ``size``.

    forward: pad to 2*size, FFT, transfer function x band limit x aperture,
    inverse FFT, centred crop (python_function.py:111-163); backward is the
    exact adjoint (python_function.py:166-218).
    """

    @staticmethod
    def forward(ctx, field: torch.Tensor, wavelength: float, pixel_pitch: float,
                distance: float, size: Tuple[int, int], aperture_size: float = -1.0):
        ctx.wavelength = wavelength
        ctx.pixel_pitch = pixel_pitch
        ctx.distance = distance
        ctx.input_size = tuple(field.shape[-2:])
        ctx.target_size = size
        ctx.aperture_size = aperture_size
        return _prop.propagate(field, wavelength, pixel_pitch, distance, size, aperture_size)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        grad = _prop.propagate_adjoint(grad_output, ctx.input_size, ctx.wavelength,
                                       ctx.pixel_pitch, ctx.distance, ctx.target_size,
                                       ctx.aperture_size)
        return grad, None, None, None, None, None


def BandlimitedPropagation(field: torch.Tensor, wavelength: float, pixel_pitch: float,
                           distance: float, size: Tuple[int, int], use_cuda: bool,
                           aperture_size: float = -1.0) -> torch.Tensor:
    """python_function.py:220-226.  ``use_cuda=True`` is the accelerated path.

    ``use_cuda=False`` selects the reference's separate pure-PyTorch ASM
    (python_function.py:35-78, float32 kz and an odak aperture mask); that
    algorithm is not part of this library and raises.
    """
    if not use_cuda:
        raise NotImplementedError(
            "BandlimitedPropagation(use_cuda=False) is the reference's pure-PyTorch ASM; "
            "this library implements the accelerated path only (use_cuda=True)")
    return BandlimitedPropagationFunction.apply(field, wavelength, pixel_pitch, distance, size,
                                                aperture_size)


class MultiPlanePropagationFunction(Function):
    """All planes and wavelengths in one call: fields (P,C,H,W) -> hologram
    (C,S,S) with hologram[c] = sum_p BandlimitedPropagation(fields[p,c],
    wavelengths[c], pitch, distances[p], size, aperture) (the loop and Python
    sum of Scene.splat, model.py:1251-1272)."""

    @staticmethod
    def forward(ctx, fields, wavelengths, pixel_pitch, distances, size, aperture_size=-1.0):
        ctx.args = (tuple(fields.shape[-2:]), wavelengths, pixel_pitch, distances, size,
                    aperture_size)
        return _prop.multiplane(fields, wavelengths, pixel_pitch, distances, size,
                                aperture_size)

    @staticmethod
    def backward(ctx, grad_hologram):
        hw, wavelengths, pixel_pitch, distances, size, aperture_size = ctx.args
        grad = _prop.multiplane_adjoint(grad_hologram, hw, wavelengths, pixel_pitch, distances,
                                        size, aperture_size)
        return grad, None, None, None, None, None


def multiplane_propagation(fields, wavelengths, pixel_pitch, distances, size,
                           aperture_size=-1.0):
    return MultiPlanePropagationFunction.apply(fields, wavelengths, pixel_pitch, distances,
                                               size, aperture_size)


def compute_bmm_cuda(diff: torch.Tensor, cov_inv: torch.Tensor) -> torch.Tensor:
    """(N,HW,2) x (N,2,2) -> (N,HW,2), out_j = sum_i diff_i cov_inv[i][j]
    (batch_matrix_mult_cuda.cu:48-49).  Helper of the reference's Python
    fallback splat only; evaluated with torch on the tensors' device."""
    return torch.matmul(diff, cov_inv.contiguous())


def sum_last_dim_cuda(x: torch.Tensor) -> torch.Tensor:
    """(N,HW,2) -> (N,HW), x0 + x1 (sum_last_dim_cuda.cu:39)."""
    if x.dim() != 3 or x.shape[-1] != 2:
        raise ValueError(f"Input must be (N, HW, 2), but got {x.shape}")
    return x[..., 0] + x[..., 1]


def element_wise_multiplication_cuda(input1: torch.Tensor, input2: torch.Tensor) -> torch.Tensor:
    """Elementwise product of two (N,HW,2) tensors (element_wise_mult_cuda.cu:34-35)."""
    assert input1.dim() == 3 and input1.shape[-1] == 2, "input1 must be (N, HW, 2)"
    assert input2.dim() == 3 and input2.shape[-1] == 2, "input2 must be (N, HW, 2)"
    assert input1.shape[:2] == input2.shape[:2], "input1 and input2 dimensions must match"
    return input1 * input2
