"""Seeded synthetic scenes for the benchmark configurations.

Each scene is produced as the reference's caller would hand it to the
rasterizer (Scene.render, model.py:1365-1416): camera-space means
X_cam = X_world @ R + T (pytorch3d convention, model.py:1105-1113),
z = X_cam[:, 2], the near/far filter, an ascending (stable) depth sort, and
post-activation parameters (normalised quaternions, exp scales, phase in
[0, 2pi), sigmoid opacity, one-hot plane assignment, model.py:41-56,594-608).

Random draws use numpy PCG64 with seed 1000 + config index, in the order
means, log-scales, quaternions, amplitude, phase, plane logits, then the
upstream gradient.  Physics constants follow the reference's training
setup (train.py:839-865): pitch 3.74 um, pad_size = aperture = max(W, H).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List

import numpy as np

PITCH = 3.74e-6
NEAR = 1.0
FAR = 1000.0
RGB = [639e-9, 515e-9, 473e-9]


@dataclass
class SceneSpec:
    name: str
    index: int
    n: int
    width: int
    height: int
    planes: int
    wavelengths: List[float]
    distances: List[float]  # args_prop.distances; propagation uses -distances[p]
    layout: str = "object"  # object | uniform | frustum | stress
    log_scale_mean: float = -4.0
    log_scale_std: float = 0.5
    backward: bool = True

    @property
    def size(self) -> int:
        return max(self.width, self.height)


def _linspace_f32(a: float, b: float, n: int) -> List[float]:
    import torch

    return [float(v) for v in torch.linspace(a, b, n, dtype=torch.float32)]


def config(name: str) -> SceneSpec:
    if name in ("cfg0", "0"):
        return SceneSpec("cfg0", 0, 10_000, 256, 256, 1, [515e-9], [-2e-3], "uniform",
                         backward=False)
    if name in ("cfg1", "1"):
        return SceneSpec("cfg1", 1, 300_000, 800, 800, 3, RGB, _linspace_f32(-1e-3, 1e-3, 3),
                         "object")
    if name in ("headline", "h"):
        return SceneSpec("headline", 1, 1_000_000, 800, 800, 3, RGB,
                         _linspace_f32(-1e-3, 1e-3, 3), "object")
    if name in ("cfg2", "2"):
        return SceneSpec("cfg2", 2, 1_000_000, 1008, 756, 6, RGB, _linspace_f32(0.0, 5e-3, 6),
                         "frustum", -5.0, 0.7)
    if name in ("cfg4", "4"):
        return SceneSpec("cfg4", 4, 3_000_000, 1920, 1080, 3, RGB,
                         _linspace_f32(-1e-3, 1e-3, 3), "stress")
    raise KeyError(name)


def small(name: str, n: int, width: int, height: int, planes: int, channels: int,
          layout: str = "uniform", seed: int = 7) -> SceneSpec:
    """A reduced scene for parity tests (same generator, custom sizes)."""
    wl = RGB[:channels] if channels > 1 else [515e-9]
    ds = _linspace_f32(-1e-3, 1e-3, planes) if planes > 1 else [-2e-3]
    return SceneSpec(name, seed - 1000, n, width, height, planes, wl, ds, layout)


@dataclass
class Scene:
    spec: SceneSpec
    cam_means: np.ndarray
    z: np.ndarray
    quats: np.ndarray
    scales: np.ndarray
    colours: np.ndarray
    phase: np.ndarray
    opac: np.ndarray
    pprobs: np.ndarray
    fx: float
    fy: float
    px: float
    py: float
    view: np.ndarray
    grad_holo: np.ndarray = field(default=None)
    n_generated: int = 0
    counts: dict = field(default_factory=dict)


def _camera(spec: SceneSpec):
    W, H = spec.width, spec.height
    f = (W / 2.0) / math.tan(math.radians(25.0))
    if spec.layout == "frustum":
        R = np.eye(3, dtype=np.float32)
        T = np.zeros(3, np.float32)
    else:
        R = np.diag([-1.0, 1.0, -1.0]).astype(np.float32)
        T = np.array([0.0, 0.0, 4.0], np.float32)
    return R, T, np.float32(f), np.float32(f), np.float32(W / 2.0), np.float32(H / 2.0)


def _draw(spec: SceneSpec, rng):
    """World-space means and post-activation parameters of all spec.n
    Gaussians, drawn from rng in a fixed order."""
    n = spec.n
    W, H = spec.width, spec.height
    counts = {}
    # means
    if spec.layout == "uniform":
        means = rng.uniform(-1.0, 1.0, size=(n, 3))
    elif spec.layout == "object":
        means = rng.normal(0.0, 0.6, size=(n, 3))
    elif spec.layout == "frustum":
        z = rng.uniform(2.0, 10.0, size=n)
        u = rng.uniform(-1.0, 1.0, size=n)
        v = rng.uniform(-1.0, 1.0, size=n)
        t = math.tan(math.radians(25.0))
        means = np.stack([u * z * t, v * z * t * H / W, z], axis=1)
    elif spec.layout == "stress":
        kind = rng.uniform(size=n)
        inside = rng.uniform(-1.0, 1.0, size=(n, 3))
        behind = np.stack([rng.uniform(-1, 1, n), rng.uniform(-1, 1, n),
                           rng.uniform(3.5, 6.0, n)], axis=1)
        side = rng.choice([-1.0, 1.0], size=n) * rng.uniform(3.0, 6.0, size=n)
        lateral = np.stack([side, rng.uniform(-1, 1, n), rng.uniform(-1, 1, n)], axis=1)
        means = np.where((kind < 0.3)[:, None], behind,
                         np.where((kind < 0.6)[:, None], lateral, inside))
        counts = {"behind": int((kind < 0.3).sum()),
                  "lateral": int(((kind >= 0.3) & (kind < 0.6)).sum()),
                  "inside": int((kind >= 0.6).sum())}
    else:
        raise ValueError(spec.layout)
    means = means.astype(np.float32)
    # log-scales
    if spec.layout == "stress":
        ls = rng.normal(-6.0, 0.5, size=(n, 3))
        ls[:, 0] = rng.normal(-2.0, 0.5, size=n)
    else:
        ls = rng.normal(spec.log_scale_mean, spec.log_scale_std, size=(n, 3))
    scales = np.exp(ls).astype(np.float32)
    q = rng.normal(size=(n, 4))
    q = q / np.maximum(np.linalg.norm(q, axis=1, keepdims=True), 1e-12)
    quats = q.astype(np.float32)
    C = len(spec.wavelengths)
    colours = rng.uniform(0.0, 1.0, size=(n, C)).astype(np.float32)
    phase = rng.uniform(0.0, 2.0 * math.pi, size=(n, C)).astype(np.float32)
    logits = rng.normal(size=(n, spec.planes)) * 10.0
    pprobs = np.eye(spec.planes, dtype=np.float32)[np.argmax(logits, axis=1)]
    opac = np.full(n, 1.0 / (1.0 + math.exp(-1.0)), np.float32)
    return dict(means=means, ls=ls, scales=scales, quats=quats, colours=colours, phase=phase,
                logits=logits, pprobs=pprobs, opac=opac, counts=counts)


def generate(spec: SceneSpec, with_grad: bool = True) -> Scene:
    rng = np.random.default_rng(1000 + spec.index)
    n = spec.n
    C = len(spec.wavelengths)
    d = _draw(spec, rng)
    means, scales, quats, colours = d["means"], d["scales"], d["quats"], d["colours"]
    phase, pprobs, opac, counts = d["phase"], d["pprobs"], d["opac"], d["counts"]
    R, T, fx, fy, px, py = _camera(spec)
    cam = (means @ R + T).astype(np.float32)
    z = cam[:, 2].copy()
    keep = np.nonzero((z > NEAR) & (z < FAR))[0]
    order = keep[np.argsort(z[keep], kind="stable")]
    sc = Scene(spec=spec, cam_means=np.ascontiguousarray(cam[order]),
               z=np.ascontiguousarray(z[order]), quats=np.ascontiguousarray(quats[order]),
               scales=np.ascontiguousarray(scales[order]),
               colours=np.ascontiguousarray(colours[order]),
               phase=np.ascontiguousarray(phase[order]), opac=np.ascontiguousarray(opac[order]),
               pprobs=np.ascontiguousarray(pprobs[order]), fx=float(fx), fy=float(fy),
               px=float(px), py=float(py), view=np.ascontiguousarray(R, np.float32),
               n_generated=n, counts=counts)
    if with_grad:
        S = spec.size
        g = (rng.normal(size=(C, S, S)) + 1j * rng.normal(size=(C, S, S))) * math.sqrt(0.5)
        sc.grad_holo = g.astype(np.complex64)
    return sc


def generate_params(spec: SceneSpec) -> dict:
    """The same Gaussians as generate(spec), as the model's parameters before
    Scene.render: world-space means, pre-activation quats (unnormalised),
    log-scales, colours, phase (shifted by whole turns), opacity and
    plane-assignment logits, all N rows unsorted, plus the camera R, T.
    render_preprocess of these gives generate(spec)'s inputs up to rounding."""
    rng = np.random.default_rng(1000 + spec.index)
    n = spec.n
    d = _draw(spec, rng)
    R, T, _, _, _, _ = _camera(spec)
    extra = np.random.default_rng(7000 + spec.index)
    C = d["colours"].shape[1]
    f32 = lambda a: np.ascontiguousarray(a, np.float32)  # noqa: E731
    return dict(
        means=f32(d["means"]),
        pre_quats=f32(d["quats"] * extra.uniform(0.5, 2.0, size=(n, 1))),
        pre_scales=f32(d["ls"]),
        colours=f32(d["colours"]),
        pre_phase=f32(d["phase"] + 2.0 * math.pi * extra.integers(-2, 3, size=(n, C))),
        pre_opac=np.ones(n, np.float32),
        pre_plane=f32(d["logits"]),
        R=f32(R), T=f32(T))


def cfg3_fields(size: int = 2048, channels: int = 3, seed: int = 3):
    """Config 3, the propagation-only microbench: a seeded complex64 field
    (C, size, size) with amplitude U(0,1) and phase U(0, 2 pi), the RGB
    wavelengths, and 8 distances log-spaced over 0.1-10 mm; 2x padding, so
    the grid is 2*size."""
    rng = np.random.default_rng(1000 + seed)
    amp = rng.uniform(0.0, 1.0, size=(channels, size, size))
    ph = rng.uniform(0.0, 2.0 * math.pi, size=(channels, size, size))
    field = (amp * np.exp(1j * ph)).astype(np.complex64)
    distances = [float(np.float32(v)) for v in np.logspace(-4, -2, 8)]
    return field, RGB[:channels], distances


def to_torch(sc: Scene, device="cuda"):
    """Scene -> dict of torch tensors on ``device`` (float32)."""
    import torch

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    out = dict(cam_means=t(sc.cam_means), z=t(sc.z), quats=t(sc.quats), scales=t(sc.scales),
               colours=t(sc.colours), phase=t(sc.phase), opac=t(sc.opac), pprobs=t(sc.pprobs),
               view=t(sc.view))
    if sc.grad_holo is not None:
        out["grad_holo"] = t(sc.grad_holo)
    return out
