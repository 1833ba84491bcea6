"""Drop-in for ``cuda_prop/cov3d_cuda/python_import.py`` of the reference.

``SplatTileCuda`` / ``splat_tile_cuda`` keep the reference signature and
tuple order (python_import.py:283-342,421-447); ``Rasterizer`` keeps the
pybind class interface (binding.cpp:31-36, rasterizer_splat.h:255-293).
The geometry operators ``compute_cov3d_cuda``, ``compute_jacobian_cuda``,
``compute_cov2d_cuda``, ``compute_means2d_cuda`` and ``invert_cov2d_cuda``
(python_import.py:53-281,343-419) are here too: ``model.py:16-19`` imports
them in the same statement as ``splat_tile_cuda``.  So are ``fast_ssim``
(with ``FusedSSIMMap``, ``C1``, ``C2``; python_import.py:43-58,449-454) and
``sparse_adam_update`` (:457-460), which ``utils/data_utils.py:20`` and
``utils/optimizer.py:21`` import, both on HIP kernels.
Unlike the reference nothing is built at import time (python_import.py:9-16),
the forward state travels in the autograd context instead of a process-wide
singleton (so two forwards before one backward are safe), and every error
raises.
"""
from __future__ import annotations

from torch.autograd import Function

from ... import geometry as _geom
from ... import rasterizer as _rast
from ...optim import sparse_adam_update  # noqa: F401  (python_import.py:457-460)
from ...ssim import FusedSSIMMap  # noqa: F401  (python_import.py:43-58)


class Rasterizer:
    """Stateless stand-in for the pybind ``Rasterizer`` class."""

    def forward(self, cam_means_3D, z_vals, quats, scales, colours, phase, opacities,
                plane_probs, fx, fy, px, py, view_matrix, img_size, tile_size, near_plane,
                far_plane):
        return _rast.forward(cam_means_3D, z_vals, quats, scales, colours, phase, opacities,
                             plane_probs, fx, fy, px, py, view_matrix, img_size, tile_size,
                             near_plane, far_plane)

    def backward(self, grad_output, cam_means_3D, z_vals, quats, scales, colours, phase,
                 opacities, plane_probs, fx, fy, px, py, view_matrix, img_size, tile_size,
                 final_Ts, n_contrib, point_list, ranges, near_plane, far_plane):
        return _rast.backward(grad_output, cam_means_3D, z_vals, quats, scales, colours, phase,
                              opacities, plane_probs, fx, fy, px, py, view_matrix, img_size,
                              tile_size, final_Ts, n_contrib, point_list, ranges, near_plane,
                              far_plane)


cuda_rasterizer = None


def get_rasterizer() -> Rasterizer:
    global cuda_rasterizer
    if cuda_rasterizer is None:
        cuda_rasterizer = Rasterizer()
    return cuda_rasterizer


class SplatTileCuda(Function):
    @staticmethod
    def forward(ctx, cam_means_3D, z_vals, quats, scales, colours, phase, opacities,
                plane_probs, fx, fy, px, py, view_matrix, img_size, near_plane, far_plane,
                tile_size=(16, 16)):
        ctx.save_for_backward(cam_means_3D, z_vals, quats, scales, colours, phase, opacities,
                              plane_probs, view_matrix)
        ctx.fx, ctx.fy, ctx.px, ctx.py = fx, fy, px, py
        ctx.img_size = img_size
        ctx.tile_size = tile_size
        ctx.near_plane = near_plane
        ctx.far_plane = far_plane
        # The forward's render records travel with the context, so the
        # backward does not recompute the projection.
        output, forward_info, ctx.geometry = _rast.forward(
            cam_means_3D, z_vals, quats, scales, colours, phase, opacities, plane_probs, fx, fy,
            px, py, view_matrix, img_size, tile_size, near_plane, far_plane, keep_geometry=True)
        ctx.forward_info = forward_info
        visible_indices = forward_info[-1]
        ctx.mark_non_differentiable(visible_indices)
        return output, visible_indices

    @staticmethod
    def backward(ctx, grad_output, grad_visible_indices=None):
        (cam_means_3D, z_vals, quats, scales, colours, phase, opacities, plane_probs,
         view_matrix) = ctx.saved_tensors
        final_Ts, n_contrib, point_list, ranges, _visible = ctx.forward_info
        grads = _rast.backward(
            grad_output.contiguous(), cam_means_3D, z_vals, quats, scales, colours, phase,
            opacities, plane_probs, ctx.fx, ctx.fy, ctx.px, ctx.py, view_matrix, ctx.img_size,
            ctx.tile_size, final_Ts, n_contrib, point_list, ranges, ctx.near_plane,
            ctx.far_plane, geometry=ctx.geometry)
        ctx.geometry = None
        return (*grads, None, None, None, None, None, None, None, None, None)


def splat_tile_cuda(cam_means_3D, z_vals, quats, scales, colours, phase, opacities,
                    plane_probs, fx, fy, px, py, view_matrix, img_size, near_plane, far_plane,
                    tile_size=(16, 16)):
    """Tile-based complex Gaussian splatting -> (field (P,C,H,W) complex64,
    visible_indices int64)."""
    return SplatTileCuda.apply(cam_means_3D, z_vals, quats, scales, colours, phase, opacities,
                               plane_probs, fx, fy, px, py, view_matrix, img_size, near_plane,
                               far_plane, tile_size)


def _require_cuda(*tensors):
    # The reference's operators raise ValueError for host tensors
    # (python_import.py:74-75 and the other forwards).
    if not all(t.is_cuda for t in tensors):
        raise ValueError("Inputs must be CUDA tensors")


class Compute3DCovarianceFunction(Function):
    """Sigma = R S^2 R^T (N,3,3) with the reference's backward."""

    @staticmethod
    def forward(ctx, quats, scales):
        quats, scales = quats.contiguous(), scales.contiguous()
        _require_cuda(quats, scales)
        ctx.save_for_backward(quats, scales)
        return _geom.cov3d_forward(quats, scales)

    @staticmethod
    def backward(ctx, grad_output):
        quats, scales = ctx.saved_tensors
        gq, gs = _geom.cov3d_backward(grad_output.contiguous(), quats, scales)
        return gq, gs


class ComputeJacobianFunction(Function):
    """Projection Jacobian (N,2,3); img_size = (width, height)."""

    @staticmethod
    def forward(ctx, cam_means_3D, fx, fy, img_size, near_plane, far_plane):
        cam_means_3D = cam_means_3D.contiguous()
        _require_cuda(cam_means_3D)
        ctx.save_for_backward(cam_means_3D)
        ctx.args = (fx, fy, int(img_size[0]), int(img_size[1]), near_plane, far_plane)
        return _geom.jacobian_forward(cam_means_3D, *ctx.args)

    @staticmethod
    def backward(ctx, grad_output):
        (cam_means_3D,) = ctx.saved_tensors
        g = _geom.jacobian_backward(grad_output.contiguous(), cam_means_3D, *ctx.args)
        return g, None, None, None, None, None


class ComputeCov2DFunction(Function):
    """cov2D (N,2,2); saves J, Sigma, W, JW for the reference's backward."""

    @staticmethod
    def forward(ctx, cam_means_3D, quats, scales, view_matrix, fx, fy, img_size, near_plane,
                far_plane):
        cam_means_3D, quats = cam_means_3D.contiguous(), quats.contiguous()
        scales, view_matrix = scales.contiguous(), view_matrix.contiguous()
        _require_cuda(cam_means_3D, quats, scales, view_matrix)
        width, height = int(img_size[0]), int(img_size[1])
        cov2d, J, cov3D, W, JW = _geom.cov2d_forward(cam_means_3D, quats, scales, view_matrix,
                                                    fx, fy, width, height, near_plane,
                                                    far_plane)
        ctx.save_for_backward(cam_means_3D, quats, scales, view_matrix, J, cov3D, W, JW)
        ctx.args = (fx, fy, width, height, near_plane, far_plane)
        return cov2d

    @staticmethod
    def backward(ctx, grad_output):
        cam_means_3D, quats, scales, view_matrix, J, cov3D, W, JW = ctx.saved_tensors
        gc, gq, gs = _geom.cov2d_backward(grad_output.contiguous(), cam_means_3D, quats, scales,
                                          view_matrix, J, cov3D, W, JW, *ctx.args)
        return gc, gq, gs, None, None, None, None, None, None


class ComputeMeans2DFunction(Function):
    """Pinhole projection (N,2); clipped points map to (1e6, 1e6)."""

    @staticmethod
    def forward(ctx, cam_means_3D, fx, fy, px, py, near_plane, far_plane):
        cam_means_3D = cam_means_3D.contiguous()
        _require_cuda(cam_means_3D)
        ctx.save_for_backward(cam_means_3D)
        ctx.args = (fx, fy, px, py, near_plane, far_plane)
        return _geom.means2d_forward(cam_means_3D, *ctx.args)

    @staticmethod
    def backward(ctx, grad_output):
        (cam_means_3D,) = ctx.saved_tensors
        g = _geom.means2d_backward(grad_output.contiguous(), cam_means_3D, *ctx.args)
        return g, None, None, None, None, None, None


class InvertCov2DFunction(Function):
    """Batched 2x2 inverse."""

    @staticmethod
    def forward(ctx, cov_2D):
        cov_2D = cov_2D.contiguous()
        _require_cuda(cov_2D)
        ctx.save_for_backward(cov_2D)
        return _geom.invert_cov2d_forward(cov_2D)

    @staticmethod
    def backward(ctx, grad_output):
        (cov_2D,) = ctx.saved_tensors
        return _geom.invert_cov2d_backward(grad_output.contiguous(), cov_2D)


def compute_cov3d_cuda(quats, scales):
    """(N,4), (N,3) -> (N,3,3)."""
    return Compute3DCovarianceFunction.apply(quats, scales)


def compute_jacobian_cuda(cam_means_3D, fx, fy, img_size, near_plane, far_plane):
    """(N,3) -> (N,2,3)."""
    return ComputeJacobianFunction.apply(cam_means_3D, fx, fy, img_size, near_plane, far_plane)


def compute_cov2d_cuda(cam_means_3D, quats, scales, view_matrix, fx, fy, img_size, near_plane,
                       far_plane):
    """-> (N,2,2)."""
    return ComputeCov2DFunction.apply(cam_means_3D, quats, scales, view_matrix, fx, fy,
                                      img_size, near_plane, far_plane)


def compute_means2d_cuda(cam_means_3D, fx, fy, px, py, near_plane, far_plane):
    """(N,3) -> (N,2)."""
    return ComputeMeans2DFunction.apply(cam_means_3D, fx, fy, px, py, near_plane, far_plane)


def invert_cov2d_cuda(cov_2D):
    """(N,2,2) -> (N,2,2)."""
    return InvertCov2DFunction.apply(cov_2D)


# SSIM constants and loss of python_import.py:449-454.
C1 = 0.01 ** 2
C2 = 0.03 ** 2


def fast_ssim(img1, img2):
    """Mean of the fused SSIM map of two (C, H, W) images."""
    ssim_map = FusedSSIMMap.apply(C1, C2, img1, img2)
    return ssim_map.mean()

