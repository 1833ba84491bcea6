"""Standalone per-Gaussian geometry operators on the HIP library.

Mirrors the reference's ``cov3d_cuda`` bindings (binding.cpp:14-25;
wave_rasterizer/forward.cu:138-432, backward.cu:274-627): the same inputs,
output shapes and shape checks (``TORCH_CHECK`` -> RuntimeError).  The
rasterizer does not use these (its projection is fused); they back the
``compute_*_cuda`` autograd operators of the compat module.
"""
from __future__ import annotations

from typing import List, Tuple

import torch

from . import _lib


def _chk(t: torch.Tensor, name: str, shape: Tuple[int, ...], n: int | None = None) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if t.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32 (got {t.dtype})")
    if t.dim() != len(shape) + 1 or tuple(t.shape[1:]) != shape:
        raise RuntimeError(f"{name} must have shape (N, {', '.join(map(str, shape))}); "
                           f"got {tuple(t.shape)}")
    if n is not None and t.shape[0] != n:
        raise RuntimeError(f"{name} has batch {t.shape[0]}, expected {n}")
    return t.contiguous()


def _view(vm: torch.Tensor) -> torch.Tensor:
    if not isinstance(vm, torch.Tensor) or not vm.is_cuda:
        raise RuntimeError("view_matrix must be a CUDA tensor")
    if tuple(vm.shape) != (3, 3):
        raise RuntimeError(f"view_matrix must have shape (3, 3); got {tuple(vm.shape)}")
    return vm.to(torch.float32).contiguous()


def _s(t: torch.Tensor) -> int:
    return _lib.stream_ptr(t.device)


def _empty(n: int, shape, like: torch.Tensor) -> torch.Tensor:
    return torch.empty((n,) + tuple(shape), dtype=torch.float32, device=like.device)


def cov3d_forward(quats: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """(N,4), (N,3) -> Sigma (N,3,3).  forward.cu:138-181."""
    q = _chk(quats, "quats", (4,))
    s = _chk(scales, "scales", (3,), q.shape[0])
    n = q.shape[0]
    out = _empty(n, (3, 3), q)
    _lib.check(_lib.load().hrf_cov3d_forward(q.data_ptr(), s.data_ptr(), n, out.data_ptr(), _s(q)))
    return out


def cov3d_backward(grad_cov3d, quats, scales) -> List[torch.Tensor]:
    """-> [grad_quats (N,4), grad_scales (N,3)].  backward.cu:274-320."""
    q = _chk(quats, "quats", (4,))
    n = q.shape[0]
    g = _chk(grad_cov3d, "grad_cov3d", (3, 3), n)
    s = _chk(scales, "scales", (3,), n)
    gq, gs = _empty(n, (4,), q), _empty(n, (3,), q)
    _lib.check(_lib.load().hrf_cov3d_backward(g.data_ptr(), q.data_ptr(), s.data_ptr(), n,
                                              gq.data_ptr(), gs.data_ptr(), _s(q)))
    return [gq, gs]


def jacobian_forward(cam_means_3D, fx, fy, width, height, near_plane, far_plane) -> torch.Tensor:
    """(N,3) -> J (N,2,3).  forward.cu:183-219."""
    c = _chk(cam_means_3D, "cam_means_3D", (3,))
    n = c.shape[0]
    out = _empty(n, (2, 3), c)
    _lib.check(_lib.load().hrf_jacobian_forward(c.data_ptr(), n, float(fx), float(fy), int(width),
                                                int(height), float(near_plane), float(far_plane),
                                                out.data_ptr(), _s(c)))
    return out


def jacobian_backward(grad_output, cam_means_3D, fx, fy, width, height, near_plane,
                      far_plane) -> torch.Tensor:
    """dL/dJ (N,2,3) -> grad_cam (N,3).  backward.cu:322-361."""
    c = _chk(cam_means_3D, "cam_means_3D", (3,))
    n = c.shape[0]
    g = _chk(grad_output, "grad_output", (2, 3), n)
    out = _empty(n, (3,), c)
    _lib.check(_lib.load().hrf_jacobian_backward(g.data_ptr(), c.data_ptr(), n, float(fx),
                                                 float(fy), int(width), int(height),
                                                 float(near_plane), float(far_plane),
                                                 out.data_ptr(), _s(c)))
    return out


def cov2d_forward(cam_means_3D, quats, scales, view_matrix, fx, fy, width, height, near_plane,
                  far_plane) -> List[torch.Tensor]:
    """-> [cov2D (N,2,2), J (N,2,3), Sigma (N,3,3), W (N,3,3), JW (N,2,3)].
    forward.cu:221-294."""
    c = _chk(cam_means_3D, "cam_means_3D", (3,))
    n = c.shape[0]
    q = _chk(quats, "quats", (4,), n)
    s = _chk(scales, "scales", (3,), n)
    vm = _view(view_matrix)
    cov, J, sig, W, JW = (_empty(n, (2, 2), c), _empty(n, (2, 3), c), _empty(n, (3, 3), c),
                          _empty(n, (3, 3), c), _empty(n, (2, 3), c))
    _lib.check(_lib.load().hrf_cov2d_forward(
        c.data_ptr(), q.data_ptr(), s.data_ptr(), vm.data_ptr(), n, float(fx), float(fy),
        int(width), int(height), float(near_plane), float(far_plane), cov.data_ptr(),
        J.data_ptr(), sig.data_ptr(), W.data_ptr(), JW.data_ptr(), _s(c)))
    return [cov, J, sig, W, JW]


def cov2d_backward(grad_cov2d, cam_means_3D, quats, scales, view_matrix, J, cov3D, W, JW, fx,
                   fy, width, height, near_plane, far_plane) -> List[torch.Tensor]:
    """-> [grad_cam (N,3), grad_quats (N,4), grad_scales (N,3)].
    backward.cu:363-450 (uses the saved J, Sigma, W, JW as given)."""
    c = _chk(cam_means_3D, "cam_means_3D", (3,))
    n = c.shape[0]
    g = _chk(grad_cov2d, "grad_cov2d", (2, 2), n)
    q = _chk(quats, "quats", (4,), n)
    s = _chk(scales, "scales", (3,), n)
    vm = _view(view_matrix)
    J = _chk(J, "J", (2, 3), n)
    cov3D = _chk(cov3D, "cov3D", (3, 3), n)
    W = _chk(W, "W", (3, 3), n)
    JW = _chk(JW, "JW", (2, 3), n)
    gc, gq, gs = _empty(n, (3,), c), _empty(n, (4,), c), _empty(n, (3,), c)
    _lib.check(_lib.load().hrf_cov2d_backward(
        g.data_ptr(), c.data_ptr(), q.data_ptr(), s.data_ptr(), vm.data_ptr(), J.data_ptr(),
        cov3D.data_ptr(), W.data_ptr(), JW.data_ptr(), n, float(fx), float(fy), int(width),
        int(height), float(near_plane), float(far_plane), gc.data_ptr(), gq.data_ptr(),
        gs.data_ptr(), _s(c)))
    return [gc, gq, gs]


def means2d_forward(cam_means_3D, fx, fy, px, py, near_plane, far_plane) -> torch.Tensor:
    """(N,3) -> means2D (N,2).  forward.cu:358-394."""
    c = _chk(cam_means_3D, "cam_means_3D", (3,))
    n = c.shape[0]
    out = _empty(n, (2,), c)
    _lib.check(_lib.load().hrf_means2d_forward(c.data_ptr(), n, float(fx), float(fy), float(px),
                                               float(py), float(near_plane), float(far_plane),
                                               out.data_ptr(), _s(c)))
    return out


def means2d_backward(grad_output, cam_means_3D, fx, fy, px, py, near_plane,
                     far_plane) -> torch.Tensor:
    """dL/dmeans2D (N,2) -> grad_cam (N,3).  backward.cu:545-585."""
    c = _chk(cam_means_3D, "cam_means_3D", (3,))
    n = c.shape[0]
    g = _chk(grad_output, "grad_output", (2,), n)
    out = _empty(n, (3,), c)
    _lib.check(_lib.load().hrf_means2d_backward(g.data_ptr(), c.data_ptr(), n, float(fx),
                                                float(fy), float(px), float(py),
                                                float(near_plane), float(far_plane),
                                                out.data_ptr(), _s(c)))
    return out


def invert_cov2d_forward(cov_2D) -> torch.Tensor:
    """(N,2,2) -> inverse (N,2,2).  forward.cu:396-432."""
    c = _chk(cov_2D, "cov_2D", (2, 2))
    n = c.shape[0]
    out = _empty(n, (2, 2), c)
    _lib.check(_lib.load().hrf_invert_cov2d_forward(c.data_ptr(), n, out.data_ptr(), _s(c)))
    return out


def invert_cov2d_backward(grad_output, cov_2D) -> torch.Tensor:
    """-(A^-1 G A^-1).  backward.cu:587-627."""
    c = _chk(cov_2D, "cov_2D", (2, 2))
    n = c.shape[0]
    g = _chk(grad_output, "grad_output", (2, 2), n)
    out = _empty(n, (2, 2), c)
    _lib.check(_lib.load().hrf_invert_cov2d_backward(g.data_ptr(), c.data_ptr(), n,
                                                     out.data_ptr(), _s(c)))
    return out
