"""Fused SSIM on the HIP library: the map and its gradient with respect to
the first image.

Mirrors ``fusedssim`` / ``fusedssim_backward`` of the reference's cov3d_cuda
module (cuda_prop/cov3d_cuda/conv.cu:935-1197) and the ``FusedSSIMMap``
autograd function (python_import.py:43-58): images (C, H, W) float32, an
11x11 Gaussian window (sigma 1.5) with zero padding, the stabilising
constants passed in; the second image gets no gradient.  The reference's
kernels are compiled for C = 3 only; any C >= 1 works here.
"""
from __future__ import annotations

import torch
from torch.autograd import Function

from . import _lib


def _img(t: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA tensor (the SSIM kernels have no CPU path)")
    if t.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32 (got {t.dtype})")
    if t.dim() != 3:
        raise RuntimeError(f"{name} must have shape (C, H, W); got {tuple(t.shape)}")
    return t.contiguous()


def _pair(img1: torch.Tensor, img2: torch.Tensor):
    a = _img(img1, "img1")
    b = _img(img2, "img2")
    if a.shape != b.shape or a.device != b.device:
        raise RuntimeError(f"img1 {tuple(a.shape)} and img2 {tuple(b.shape)} must match")
    return a, b


def ssim_map(C1: float, C2: float, img1: torch.Tensor, img2: torch.Tensor) -> torch.Tensor:
    """SSIM map (C, H, W) of two (C, H, W) images.  conv.cu:1138-1166."""
    a, b = _pair(img1, img2)
    C, H, W = a.shape
    out = torch.empty_like(a)
    if out.numel() == 0:
        return out
    _lib.check(_lib.load().hrf_ssim_map(a.data_ptr(), b.data_ptr(), C, H, W, float(C1),
                                        float(C2), out.data_ptr(), _lib.stream_ptr(a.device)))
    return out


def ssim_backward(C1: float, C2: float, img1: torch.Tensor, img2: torch.Tensor,
                  grad_map: torch.Tensor) -> torch.Tensor:
    """d(sum grad_map * map)/d img1, shape (C, H, W).  conv.cu:1168-1197."""
    a, b = _pair(img1, img2)
    g = _img(grad_map, "grad_map")
    if g.shape != a.shape:
        raise RuntimeError(f"grad_map {tuple(g.shape)} must match the images {tuple(a.shape)}")
    C, H, W = a.shape
    out = torch.empty_like(a)
    if out.numel() == 0:
        return out
    _lib.check(_lib.load().hrf_ssim_backward(a.data_ptr(), b.data_ptr(), g.data_ptr(), C, H, W,
                                             float(C1), float(C2), out.data_ptr(),
                                             _lib.stream_ptr(a.device)))
    return out


class FusedSSIMMap(Function):
    """Autograd function of the SSIM map (python_import.py:43-58)."""

    @staticmethod
    def forward(ctx, C1, C2, img1, img2):
        m = ssim_map(C1, C2, img1, img2)
        ctx.save_for_backward(img1.detach(), img2)
        ctx.C1 = C1
        ctx.C2 = C2
        return m

    @staticmethod
    def backward(ctx, opt_grad):
        img1, img2 = ctx.saved_tensors
        grad = ssim_backward(ctx.C1, ctx.C2, img1, img2, opt_grad)
        return None, None, grad, None
