"""Drop-in for ``cuda_prop/cov3d_cuda/python_import.py`` of the reference.

``SplatTileCuda`` / ``splat_tile_cuda`` keep the reference signature and
tuple order (python_import.py:283-342,421-447); ``Rasterizer`` keeps the
pybind class interface (binding.cpp:31-36, rasterizer_splat.h:255-293).
Unlike the reference nothing is built at import time (python_import.py:9-16),
the forward state travels in the autograd context instead of a process-wide
singleton (so two forwards before one backward are safe), and every error
raises.
"""
from __future__ import annotations

from torch.autograd import Function

from ... import rasterizer as _rast


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
        output, forward_info = get_rasterizer().forward(
            cam_means_3D, z_vals, quats, scales, colours, phase, opacities, plane_probs, fx, fy,
            px, py, view_matrix, img_size, tile_size, near_plane, far_plane)
        ctx.forward_info = forward_info
        visible_indices = forward_info[-1]
        ctx.mark_non_differentiable(visible_indices)
        return output, visible_indices

    @staticmethod
    def backward(ctx, grad_output, grad_visible_indices=None):
        (cam_means_3D, z_vals, quats, scales, colours, phase, opacities, plane_probs,
         view_matrix) = ctx.saved_tensors
        final_Ts, n_contrib, point_list, ranges, _visible = ctx.forward_info
        grads = get_rasterizer().backward(
            grad_output.contiguous(), cam_means_3D, z_vals, quats, scales, colours, phase,
            opacities, plane_probs, ctx.fx, ctx.fy, ctx.px, ctx.py, view_matrix, ctx.img_size,
            ctx.tile_size, final_Ts, n_contrib, point_list, ranges, ctx.near_plane,
            ctx.far_plane)
        return (*grads, None, None, None, None, None, None, None, None, None)


def splat_tile_cuda(cam_means_3D, z_vals, quats, scales, colours, phase, opacities,
                    plane_probs, fx, fy, px, py, view_matrix, img_size, near_plane, far_plane,
                    tile_size=(16, 16)):
    """Tile-based complex Gaussian splatting -> (field (P,C,H,W) complex64,
    visible_indices int64)."""
    return SplatTileCuda.apply(cam_means_3D, z_vals, quats, scales, colours, phase, opacities,
                               plane_probs, fx, fy, px, py, view_matrix, img_size, near_plane,
                               far_plane, tile_size)
