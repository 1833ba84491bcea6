"""Fused render preprocess: the caller-side glue of ``Scene.render``.

Mirrors what the reference does between the model's parameters and
``splat_tile_cuda`` (model.py:1365-1402, with the world-to-view transform of
``Scene.splat``, model.py:1161-1162):

* camera-space means X @ R + T (``compute_depth_values``, model.py:1105-1112;
  pytorch3d's ``transform_points`` computes the same product) and their z;
* keep near < z < far (model.py:1382-1385) and z >= 0
  (``get_idxs_to_filter_and_sort``, model.py:1121-1125), in ascending depth
  order — stable here (ties keep the parameter order); torch.sort leaves the
  order of equal depths unspecified;
* the gathers and ``Gaussians.apply_activations`` (model.py:594-608):
  exp(log-scales), F.normalize(quats), phase mod 2*pi, sigmoid(opacities) and
  the straight-through one_hot(argmax) plane assignment (``STEFunction``,
  model.py:41-56, whose backward is grad * softmax(logits / 0.001)).

The forward runs a selection kernel over the parameters in index order (it
also computes every activation into one packed record per kept row), the
binning's flag scan and radix sort, and one gather of the records in depth
order (``include/hrf.h``: hrf_preprocess_*), with one host sync for the
selected count, as the reference's ``torch.where`` / ``masked_select`` have.
The backward packs the output gradients in depth order and then writes the
parameter gradients in index order.
"""
from __future__ import annotations

import ctypes

import torch
from torch.autograd import Function

from . import _lib

PLANE_STE_TEMPERATURE = 0.001  # STEFunction default (model.py:42)


def _f32(t: torch.Tensor, name: str, cols: int | None) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (the HIP preprocess has no CPU path)")
    if t.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32 (got {t.dtype})")
    if cols is not None and (t.dim() != 2 or t.shape[1] != cols):
        raise RuntimeError(f"{name} must have shape (N, {cols}), got {tuple(t.shape)}")
    return t.contiguous()


class _Params:
    def __init__(self, means, pre_quats, pre_scales, colours, pre_phase, pre_opac, pre_plane):
        self.means = _f32(means, "means", 3)
        n = self.means.shape[0]
        self.pre_quats = _f32(pre_quats, "pre_act_quats", 4)
        self.pre_scales = _f32(pre_scales, "pre_act_scales", 3)
        if colours.dim() != 2 or pre_phase.dim() != 2 or pre_plane.dim() != 2:
            raise RuntimeError("colours/pre_act_phase must be (N,C), pre_act_plane_assignment (N,P)")
        self.colours = _f32(colours, "colours", None)
        self.pre_phase = _f32(pre_phase, "pre_act_phase", self.colours.shape[1])
        self.pre_opac = _f32(pre_opac, "pre_act_opacities", None).reshape(-1)
        self.pre_plane = _f32(pre_plane, "pre_act_plane_assignment", None)
        for name, t in (("pre_act_quats", self.pre_quats), ("pre_act_scales", self.pre_scales),
                        ("colours", self.colours), ("pre_act_phase", self.pre_phase),
                        ("pre_act_opacities", self.pre_opac),
                        ("pre_act_plane_assignment", self.pre_plane)):
            if t.shape[0] != n:
                raise RuntimeError(f"{name} has {t.shape[0]} rows, expected {n}")
        self.n, self.C, self.P = n, int(self.colours.shape[1]), int(self.pre_plane.shape[1])
        self.device = self.means.device
        self.c = _lib.HrfSceneParams(
            self.means.data_ptr(), self.pre_quats.data_ptr(), self.pre_scales.data_ptr(),
            self.colours.data_ptr(), self.pre_phase.data_ptr(), self.pre_opac.data_ptr(),
            self.pre_plane.data_ptr(), n, self.C, self.P)


def _camera(R, T, device):
    R = R[0] if R.dim() == 3 else R
    T = T[0] if T.dim() == 2 else T
    R = _f32(R.to(device), "R", 3)
    T = _f32(T.to(device).reshape(-1), "T", None)
    if tuple(R.shape) != (3, 3) or T.numel() != 3:
        raise RuntimeError("R must be (3,3) and T (3,)")
    return R, T


def forward(means, pre_act_quats, pre_act_scales, colours, pre_act_phase, pre_act_opacities,
            pre_act_plane_assignment, R, T, near_plane=1.0, far_plane=1000.0):
    """-> (cam_means_3D (M,3), z_vals (M), quats (M,4), scales (M,3), colours (M,C),
    phase (M,C), opacities (M), plane_probs (M,P), idxs (M) int64), in ascending
    depth order; idxs are the parameter rows."""
    prm = _Params(means, pre_act_quats, pre_act_scales, colours, pre_act_phase,
                  pre_act_opacities, pre_act_plane_assignment)
    R, T = _camera(R, T, prm.device)
    lib = _lib.load()
    dev = prm.device
    with torch.cuda.device(dev):
        stream = _lib.stream_ptr(dev)
        wbytes = lib.hrf_preprocess_workspace_size(prm.n, prm.C, prm.P)
        ws = _lib.workspace("preprocess", dev, stream, wbytes)
        m = ctypes.c_int64(0)
        _lib.check(lib.hrf_preprocess_select(ctypes.byref(prm.c), R.data_ptr(), T.data_ptr(),
                                             float(near_plane), float(far_plane),
                                             _lib.ptr(ws), wbytes, stream, ctypes.byref(m)))
        m = int(m.value)
        f = dict(dtype=torch.float32, device=dev)
        out = (torch.empty((m, 3), **f), torch.empty((m,), **f), torch.empty((m, 4), **f),
               torch.empty((m, 3), **f), torch.empty((m, prm.C), **f),
               torch.empty((m, prm.C), **f), torch.empty((m,), **f),
               torch.empty((m, prm.P), **f), torch.empty((m,), dtype=torch.int64, device=dev))
        _lib.check(lib.hrf_preprocess_forward(ctypes.byref(prm.c), R.data_ptr(), T.data_ptr(),
                                              _lib.ptr(ws), wbytes, m,
                                              *[t.data_ptr() for t in out], stream))
    return out


def backward(grads, means, pre_act_quats, pre_act_scales, colours, pre_act_phase,
             pre_act_opacities, pre_act_plane_assignment, R, idxs):
    """grads: gradients of (cam_means_3D, z_vals, quats, scales, colours, phase,
    opacities, plane_probs) (z_vals may be None) -> gradients of (means,
    pre_act_quats, pre_act_scales, colours, pre_act_phase, pre_act_opacities,
    pre_act_plane_assignment), zero for rows that were not selected."""
    prm = _Params(means, pre_act_quats, pre_act_scales, colours, pre_act_phase,
                  pre_act_opacities, pre_act_plane_assignment)
    R = R[0] if R.dim() == 3 else R
    R = _f32(R.to(prm.device), "R", 3)
    idxs = idxs.contiguous()
    if idxs.dtype != torch.int64 or idxs.dim() != 1:
        raise RuntimeError("idxs must be a 1-D int64 tensor")
    m = int(idxs.numel())
    shapes = [(m, 3), (m,), (m, 4), (m, 3), (m, prm.C), (m, prm.C), (m,), (m, prm.P)]
    names = ["cam_means_3D", "z_vals", "quats", "scales", "colours", "phase", "opacities",
             "plane_probs"]
    gs = []
    for g, shp, name in zip(grads, shapes, names):
        if g is None:
            gs.append(None if name == "z_vals" else torch.zeros(shp, dtype=torch.float32,
                                                                  device=prm.device))
            continue
        g = _f32(g, "grad " + name, None).reshape(shp)
        gs.append(g)
    f = dict(dtype=torch.float32, device=prm.device)
    out = [torch.empty((prm.n, 3), **f), torch.empty((prm.n, 4), **f),
           torch.empty((prm.n, 3), **f), torch.empty((prm.n, prm.C), **f),
           torch.empty((prm.n, prm.C), **f), torch.empty((prm.n,), **f),
           torch.empty((prm.n, prm.P), **f)]
    gin = _lib.HrfSelectedGrads(*[_lib.ptr(g) for g in gs])
    gout = _lib.HrfParamGrads(*[t.data_ptr() for t in out])
    lib = _lib.load()
    with torch.cuda.device(prm.device):
        stream = _lib.stream_ptr(prm.device)
        wbytes = lib.hrf_preprocess_workspace_size(prm.n, prm.C, prm.P)
        ws = _lib.workspace("preprocess", prm.device, stream, wbytes)
        _lib.check(lib.hrf_preprocess_backward(ctypes.byref(prm.c), R.data_ptr(),
                                               idxs.data_ptr(), m, ctypes.byref(gin),
                                               ctypes.byref(gout), _lib.ptr(ws), wbytes,
                                               stream))
    out[5] = out[5].reshape(pre_act_opacities.shape)
    return out


class RenderPreprocess(Function):
    """Autograd wrapper: the 7 parameter tensors (+ R, T, near, far) -> the
    rasterizer inputs and the selected rows."""

    @staticmethod
    def forward(ctx, means, pre_act_quats, pre_act_scales, colours, pre_act_phase,
                pre_act_opacities, pre_act_plane_assignment, R, T, near_plane=1.0,
                far_plane=1000.0):
        out = forward(means, pre_act_quats, pre_act_scales, colours, pre_act_phase,
                      pre_act_opacities, pre_act_plane_assignment, R, T, near_plane, far_plane)
        ctx.save_for_backward(means, pre_act_quats, pre_act_scales, colours, pre_act_phase,
                              pre_act_opacities, pre_act_plane_assignment, R, out[-1])
        ctx.mark_non_differentiable(out[-1])
        return out

    @staticmethod
    def backward(ctx, *grads):
        (means, pq, ps, col, ph, po, pp, R, idxs) = ctx.saved_tensors
        g = backward(grads[:8], means, pq, ps, col, ph, po, pp, R, idxs)
        return (*g, None, None, None, None)


def render_preprocess(means, pre_act_quats, pre_act_scales, colours, pre_act_phase,
                      pre_act_opacities, pre_act_plane_assignment, R, T, near_plane=1.0,
                      far_plane=1000.0):
    """Differentiable drop-in for Scene.render's steps before splat
    (model.py:1377-1402 + the transform at model.py:1161-1162)."""
    return RenderPreprocess.apply(means, pre_act_quats, pre_act_scales, colours, pre_act_phase,
                                  pre_act_opacities, pre_act_plane_assignment, R, T, near_plane,
                                  far_plane)
