"""Host side of the rasterizer: torch tensors in, C-ABI calls, torch tensors out.

Mirrors ``CudaRasterizer::Rasterizer::forward/backward``
(cuda_prop/cov3d_cuda/wave_rasterizer/rasterizer_splat.h:255-293,
rasterizer_splat.cu:324-684): same arguments, same outputs, same empty-scene
behaviour, with errors raised as RuntimeError instead of printed.
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional, Sequence, Tuple

import torch

from . import _lib


def _f32c(t: torch.Tensor, name: str, shape_tail: Tuple[int, ...] | None = None) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (the HIP rasterizer has no CPU path)")
    if t.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32 (got {t.dtype})")
    if shape_tail is not None and tuple(t.shape[1:]) != shape_tail:
        raise RuntimeError(f"{name} must have shape (N, {', '.join(map(str, shape_tail))}), "
                           f"got {tuple(t.shape)}")
    return t.contiguous()


def _as_float(x) -> float:
    if isinstance(x, torch.Tensor):
        return float(x.detach().reshape(-1)[0].item())
    return float(x)


class _Inputs:
    """Validated, contiguous inputs plus the C descriptors pointing at them."""

    def __init__(self, cam_means_3D, z_vals, quats, scales, colours, phase, opacities,
                 plane_probs, fx, fy, px, py, view_matrix, img_size, near_plane, far_plane):
        self.cam = _f32c(cam_means_3D, "cam_means_3D", (3,))
        n = self.cam.shape[0]
        self.z = _f32c(z_vals, "z_vals").reshape(-1)
        self.quats = _f32c(quats, "quats", (4,))
        self.scales = _f32c(scales, "scales", (3,))
        if colours.dim() != 2 or phase.dim() != 2 or plane_probs.dim() != 2:
            raise RuntimeError("colours/phase must be (N,C) and plane_probs (N,P)")
        self.colours = _f32c(colours, "colours")
        self.phase = _f32c(phase, "phase", (self.colours.shape[1],))
        self.opac = _f32c(opacities, "opacities").reshape(-1)
        self.pprobs = _f32c(plane_probs, "plane_probs")
        for name, t in (("z_vals", self.z), ("quats", self.quats), ("scales", self.scales),
                        ("colours", self.colours), ("phase", self.phase),
                        ("opacities", self.opac), ("plane_probs", self.pprobs)):
            if t.shape[0] != n:
                raise RuntimeError(f"{name} has {t.shape[0]} rows, expected {n}")
        vm = view_matrix
        if vm.dim() == 3:
            vm = vm[0]
        self.view = _f32c(vm, "view_matrix")
        if tuple(self.view.shape) != (3, 3):
            raise RuntimeError("view_matrix must have shape (3, 3)")
        self.device = self.cam.device
        for t in (self.z, self.quats, self.scales, self.colours, self.phase, self.opac,
                  self.pprobs, self.view):
            if t.device != self.device:
                raise RuntimeError("all inputs must be on the same device")
        self.n = n
        self.C = int(self.colours.shape[1])
        self.P = int(self.pprobs.shape[1])
        self.W, self.H = int(img_size[0]), int(img_size[1])
        self.g = _lib.HrfGaussians(
            self.cam.data_ptr(), self.z.data_ptr(), self.quats.data_ptr(),
            self.scales.data_ptr(), self.colours.data_ptr(), self.phase.data_ptr(),
            self.opac.data_ptr(), self.pprobs.data_ptr(), n, self.C, self.P)
        self.c = _lib.HrfCamera(_as_float(fx), _as_float(fy), _as_float(px), _as_float(py),
                                self.view.data_ptr(), self.W, self.H, _as_float(near_plane),
                                _as_float(far_plane))

    @property
    def ntiles(self) -> int:
        return ((self.W + 15) // 16) * ((self.H + 15) // 16)


# Largest plane member list buffer (P*K*8 bytes + counts) a forward keeps for
# its backward; beyond it the backward filters the tile lists itself.
PLANE_LISTS_MAX_BYTES = 32 << 30

# The pair count of the last forward per (device, image size, Gaussian
# count): the next forward allocates its pair-sized buffers for that count
# plus an eighth before it waits for its own count, so that little host work
# lies between the count read-back and the launches that follow it.
_LAST_PAIRS: dict = {}


class ForwardGeometry(NamedTuple):
    """What forward(..., keep_geometry=True) hands to backward(geometry=):
    the geometry workspace (render records of these inputs) and the plane
    member lists of this forward's tile lists (None when not kept)."""
    workspace: torch.Tensor
    plane_lists: Optional[torch.Tensor]


def forward(cam_means_3D, z_vals, quats, scales, colours, phase, opacities, plane_probs,
            fx, fy, px, py, view_matrix, img_size: Sequence[int], tile_size=(16, 16),
            near_plane=1.0, far_plane=1000.0, keep_geometry: bool = False):
    """Rasterizer::forward -> (field (P,C,H,W) complex64,
    (final_Ts, n_contrib, point_list, ranges, visible_indices)).

    keep_geometry=True appends a third element, a ForwardGeometry: the
    forward's geometry workspace, which backward(..., geometry=) reuses
    instead of recomputing the projection, and the per-(tile, plane) member
    lists of the tile lists, which the backward walks instead of filtering
    each tile list once per plane."""
    if tuple(int(t) for t in tile_size) != (16, 16):
        # The reference ignores tile_size and always uses 16x16 tiles
        # (config.h:16-17); any other request is accepted and ignored the same way.
        pass
    inp = _Inputs(cam_means_3D, z_vals, quats, scales, colours, phase, opacities, plane_probs,
                  fx, fy, px, py, view_matrix, img_size, near_plane, far_plane)
    lib = _lib.load()
    dev = inp.device
    P, C, H, W = inp.P, inp.C, inp.H, inp.W
    with torch.cuda.device(dev):
        stream = _lib.stream_ptr(dev)
        gbytes = lib.hrf_raster_geom_workspace_size(inp.n, C, P)
        if keep_geometry:
            geom_ws = torch.empty(max(gbytes, 1), dtype=torch.uint8, device=dev)
        else:
            geom_ws = _lib.workspace("raster_geom", dev, stream, gbytes)
        # Outputs whose size does not depend on the pair count are allocated
        # before the count read-back, so little host work follows that sync.
        field = torch.empty((P, C, H, W), dtype=torch.complex64, device=dev)
        final_T = torch.empty((P, H, W), dtype=torch.float32, device=dev)
        n_contrib = torch.empty((P, H, W), dtype=torch.int32, device=dev)
        ranges = torch.empty((inp.ntiles, 2), dtype=torch.int32, device=dev)
        key = (str(dev), W, H, P, inp.n)
        last = _LAST_PAIRS.get(key, 0)
        cap = last + last // 8 + 4096 if last > 0 else 0
        if cap > 0:
            pl_buf = torch.empty(cap, dtype=torch.int32, device=dev)
            vis_buf = torch.empty(max(inp.n, 1), dtype=torch.int64, device=dev)
            cap_bbytes = lib.hrf_raster_binning_workspace_size(cap, W, H)
            cap_bin_ws = _lib.workspace("raster_bin", dev, stream, cap_bbytes)
            cap_sbytes = lib.hrf_raster_plane_lists_size(cap, W, H, P) if keep_geometry else 0
            cap_planes = (torch.empty(cap_sbytes, dtype=torch.uint8, device=dev)
                          if 0 < cap_sbytes <= PLANE_LISTS_MAX_BYTES else None)
        K = ctypes.c_int64(0)
        V = ctypes.c_int64(0)
        _lib.check(lib.hrf_raster_forward_prepare(ctypes.byref(inp.g), ctypes.byref(inp.c),
                                                  geom_ws.data_ptr(), gbytes, stream,
                                                  ctypes.byref(K), ctypes.byref(V)))
        K, V = int(K.value), int(V.value)
        _LAST_PAIRS[key] = K
        plane_lists = None
        sbytes = 0
        if K == 0:
            point_list = torch.zeros(1, dtype=torch.int32, device=dev)
            visible = torch.zeros(0, dtype=torch.int64, device=dev)
            bbytes = 0
            bin_ws = None
        elif K <= cap:
            # The buffers allocated for the last call's count hold this one.
            point_list = pl_buf[:K]
            visible = vis_buf[:V]
            bbytes, bin_ws = cap_bbytes, cap_bin_ws
            if keep_geometry and cap_planes is not None:
                plane_lists, sbytes = cap_planes, cap_sbytes
        else:
            point_list = torch.empty(K, dtype=torch.int32, device=dev)
            visible = torch.empty(V, dtype=torch.int64, device=dev)
            bbytes = lib.hrf_raster_binning_workspace_size(K, W, H)
            bin_ws = _lib.workspace("raster_bin", dev, stream, bbytes)
        if keep_geometry and K > 0 and plane_lists is None:
            sbytes = lib.hrf_raster_plane_lists_size(K, W, H, P)
            if sbytes <= PLANE_LISTS_MAX_BYTES:
                plane_lists = torch.empty(sbytes, dtype=torch.uint8, device=dev)
            else:
                sbytes = 0
        _lib.check(lib.hrf_raster_forward_render(
            ctypes.byref(inp.g), ctypes.byref(inp.c), geom_ws.data_ptr(), gbytes,
            _lib.ptr(bin_ws), bbytes, K, V if K > 0 else 0, field.data_ptr(),
            final_T.data_ptr(), n_contrib.data_ptr(), point_list.data_ptr(), ranges.data_ptr(),
            visible.data_ptr() if visible.numel() else None, _lib.ptr(plane_lists), sbytes,
            stream))
    if keep_geometry:
        return (field, (final_T, n_contrib, point_list, ranges, visible),
                ForwardGeometry(geom_ws, plane_lists))
    return field, (final_T, n_contrib, point_list, ranges, visible)


def backward_prepare(cam_means_3D, z_vals, quats, scales, colours, phase, opacities,
                     plane_probs, fx, fy, px, py, view_matrix, img_size, point_list,
                     near_plane=1.0, far_plane=1000.0,
                     geometry: ForwardGeometry | None = None, stream=None):
    """Queues the backward's prologue (accumulator clear and block order) on
    `stream` (a torch stream; default the current one) for the next
    backward(...) of these inputs on the current stream, which then waits
    for it instead of running it: the prologue can run beside the
    propagation adjoint.  The caller orders `stream` after the forward (and
    after the previous backward on this device and thread)."""
    inp = _Inputs(cam_means_3D, z_vals, quats, scales, colours, phase, opacities, plane_probs,
                  fx, fy, px, py, view_matrix, img_size, near_plane, far_plane)
    plane_lists = geometry.plane_lists if isinstance(geometry, ForwardGeometry) else None
    lib = _lib.load()
    dev = inp.device
    n, C, P = inp.n, inp.C, inp.P
    if n == 0:
        return
    with torch.cuda.device(dev):
        # the workspace the backward on the current stream will use
        wbytes = lib.hrf_raster_backward_workspace_size(n, C, P)
        ws = _lib.workspace("raster_bwd", dev, _lib.stream_ptr(dev), wbytes)
        s = stream.cuda_stream if stream is not None else _lib.stream_ptr(dev)
        _lib.check(lib.hrf_raster_backward_prepare(
            ctypes.byref(inp.g), ctypes.byref(inp.c), int(point_list.numel()), ws.data_ptr(),
            wbytes, _lib.ptr(plane_lists),
            int(plane_lists.numel()) if plane_lists is not None else 0, s))


def backward(grad_output, cam_means_3D, z_vals, quats, scales, colours, phase, opacities,
             plane_probs, fx, fy, px, py, view_matrix, img_size, tile_size, final_Ts,
             n_contrib, point_list, ranges, near_plane=1.0, far_plane=1000.0,
             geometry: ForwardGeometry | torch.Tensor | None = None):
    """Rasterizer::backward -> [grad_cam_means_3D, grad_z_vals, grad_quats, grad_scales,
    grad_colours, grad_phase, grad_opacities, grad_plane_probs].

    geometry: the ForwardGeometry forward(..., keep_geometry=True) returned
    for these same inputs and forward outputs (or just its workspace), or
    None to recompute the projection and filter the tile lists here."""
    if isinstance(geometry, ForwardGeometry):
        geom_ws, plane_lists = geometry.workspace, geometry.plane_lists
    else:
        geom_ws, plane_lists = geometry, None
    inp = _Inputs(cam_means_3D, z_vals, quats, scales, colours, phase, opacities, plane_probs,
                  fx, fy, px, py, view_matrix, img_size, near_plane, far_plane)
    lib = _lib.load()
    dev = inp.device
    n, C, P, H, W = inp.n, inp.C, inp.P, inp.H, inp.W
    go = grad_output
    if go.dtype != torch.complex64:
        go = go.to(torch.complex64)
    if tuple(go.shape) != (P, C, H, W):
        raise RuntimeError(f"grad_output must have shape {(P, C, H, W)}, got {tuple(go.shape)}")
    go = go.contiguous()
    final_Ts = final_Ts.contiguous()
    n_contrib = n_contrib.contiguous()
    point_list = point_list.contiguous()
    ranges = ranges.contiguous()
    if tuple(final_Ts.shape) != (P, H, W) or tuple(n_contrib.shape) != (P, H, W):
        raise RuntimeError("final_Ts / n_contrib must have shape (P, H, W)")
    if tuple(ranges.shape) != (inp.ntiles, 2) or ranges.dtype != torch.int32:
        raise RuntimeError(f"ranges must be int32 of shape ({inp.ntiles}, 2)")
    if point_list.dtype != torch.int32 or n_contrib.dtype != torch.int32:
        raise RuntimeError("point_list and n_contrib must be int32")
    opts = dict(dtype=torch.float32, device=dev)
    g_cam = torch.empty((n, 3), **opts)
    g_z = torch.empty((n,), **opts)
    g_q = torch.empty((n, 4), **opts)
    g_s = torch.empty((n, 3), **opts)
    g_col = torch.empty((n, C), **opts)
    g_ph = torch.empty((n, C), **opts)
    g_o = torch.empty((n,), **opts)
    g_pl = torch.empty((n, P), **opts)
    if n == 0:
        return [g_cam, g_z, g_q, g_s, g_col, g_ph, g_o, g_pl]
    with torch.cuda.device(dev):
        stream = _lib.stream_ptr(dev)
        wbytes = lib.hrf_raster_backward_workspace_size(n, C, P)
        ws = _lib.workspace("raster_bwd", dev, stream, wbytes)
        _lib.check(lib.hrf_raster_backward(
            ctypes.byref(inp.g), ctypes.byref(inp.c), go.data_ptr(), final_Ts.data_ptr(),
            n_contrib.data_ptr(), point_list.data_ptr(), ranges.data_ptr(),
            int(point_list.numel()), ws.data_ptr(), wbytes, _lib.ptr(geom_ws),
            int(geom_ws.numel()) if geom_ws is not None else 0, _lib.ptr(plane_lists),
            int(plane_lists.numel()) if plane_lists is not None else 0, g_cam.data_ptr(),
            g_z.data_ptr(),
            g_q.data_ptr(), g_s.data_ptr(), g_col.data_ptr(), g_ph.data_ptr(), g_o.data_ptr(),
            g_pl.data_ptr(), stream))
    return [g_cam, g_z, g_q, g_s, g_col, g_ph, g_o, g_pl]
