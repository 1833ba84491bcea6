"""One holographic frame on the HIP path: rasterize -> multi-plane ASM.

This is the caller the reference's Scene.splat is (model.py:1130-1274): the
rasterizer produces the (P,C,H,W) plane fields, every field is propagated to
the hologram plane with ``distance = -distances[p]`` at its wavelength, and
the planes are summed into a (C,S,S) hologram.  Backward takes the upstream
hologram gradient through the ASM adjoint and the rasterizer backward to the
8 Gaussian gradients.  Used by bench.py and smoke(); the per-(p,c) loop is a
single fused call here.
"""
from __future__ import annotations

import torch

from . import propagation, rasterizer
from .scenes import FAR, NEAR, PITCH


class Frame:
    def __init__(self, t: dict, spec, fx, fy, px, py):
        self.t = t
        self.spec = spec
        self.fx, self.fy, self.px, self.py = fx, fy, px, py
        self.img = (spec.width, spec.height)
        self.S = spec.size
        self.prop_dist = [-d for d in spec.distances]
        self.fwd_state = None
        self.fields = None
        self.geometry = None
        self._side = None  # stream of the backward prologue

    def forward(self):
        t = self.t
        field, info, geom = rasterizer.forward(
            t["cam_means"], t["z"], t["quats"], t["scales"], t["colours"], t["phase"],
            t["opac"], t["pprobs"], self.fx, self.fy, self.px, self.py, t["view"], self.img,
            (16, 16), NEAR, FAR, keep_geometry=True)
        self.fields = field
        self.fwd_state = info
        self.geometry = geom
        holo = propagation.multiplane(field, self.spec.wavelengths, PITCH, self.prop_dist,
                                      (self.S, self.S), float(self.S))
        return holo

    def backward(self, grad_holo):
        t = self.t
        final_T, n_contrib, point_list, ranges, _vis = self.fwd_state
        # The rasterizer backward's prologue (accumulator clear, block order)
        # depends only on the forward: it runs on a second stream beside the
        # propagation adjoint, and the backward waits for it.
        main = torch.cuda.current_stream(grad_holo.device)
        if self._side is None:
            self._side = torch.cuda.Stream(device=grad_holo.device)
        self._side.wait_stream(main)
        rasterizer.backward_prepare(t["cam_means"], t["z"], t["quats"], t["scales"],
                                    t["colours"], t["phase"], t["opac"], t["pprobs"], self.fx,
                                    self.fy, self.px, self.py, t["view"], self.img, point_list,
                                    NEAR, FAR, geometry=self.geometry, stream=self._side)
        gf = propagation.multiplane_adjoint(grad_holo, (self.spec.height, self.spec.width),
                                            self.spec.wavelengths, PITCH, self.prop_dist,
                                            (self.S, self.S), float(self.S))
        return rasterizer.backward(gf, t["cam_means"], t["z"], t["quats"], t["scales"],
                                   t["colours"], t["phase"], t["opac"], t["pprobs"], self.fx,
                                   self.fy, self.px, self.py, t["view"], self.img, (16, 16),
                                   final_T, n_contrib, point_list, ranges, NEAR, FAR,
                                   geometry=self.geometry)

    @property
    def num_pairs(self) -> int:
        if self.fwd_state is None:
            return 0
        rng = self.fwd_state[3]
        return int(self.fwd_state[2].numel()) if bool((rng[:, 1] > 0).any()) else 0
