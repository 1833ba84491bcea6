"""Writes the golden fixtures of this directory from the CPU oracle.

The reference ships no test vectors (no test suite, no data files), so the
fixtures are produced by the oracle (oracle/), whose functions are pinned
independently by tests/test_oracle_pinning.py (closed forms, brute force,
float64 restatements, finite differences, a brute-force DFT).  They freeze
small, fully specified cases — inputs and expected outputs — so that the
oracle cannot drift unnoticed (tests/test_golden.py) and the HIP library is
checked against fixed numbers (tests/test_gpu_golden.py).

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from complex_valued_holographic_radiance_fields_amd import scenes  # noqa: E402
from oracle import oracle as O  # noqa: E402

PITCH = 3.74e-6


def _gaussians(sc):
    return O.Gaussians(sc.cam_means, sc.z, sc.quats, sc.scales, sc.colours, sc.phase, sc.opac,
                       sc.pprobs)


def raster_fixture():
    spec = scenes.small("golden", 200, 32, 32, 2, 3, "uniform", seed=31)
    sc = scenes.generate(spec)
    g = _gaussians(sc)
    cam = O.Camera(sc.fx, sc.fy, sc.px, sc.py, sc.view, spec.width, spec.height)
    ref = O.rasterize_forward(g, cam)
    rng = np.random.default_rng(77)
    P, C, H, W = g.P, g.C, spec.height, spec.width
    gf = ((rng.normal(size=(P, C, H, W)) + 1j * rng.normal(size=(P, C, H, W))) *
          math.sqrt(0.5)).astype(np.complex64)
    rb = O.rasterize_backward(g, cam, ref, gf)
    return dict(
        cam_means=sc.cam_means, z=sc.z, quats=sc.quats, scales=sc.scales, colours=sc.colours,
        phase=sc.phase, opac=sc.opac, pprobs=sc.pprobs,
        camera=np.array([sc.fx, sc.fy, sc.px, sc.py], np.float32), view=sc.view,
        img=np.array([W, H], np.int32),
        point_list=ref["point_list"], ranges=ref["ranges"], visible=ref["visible"],
        field=ref["field"], final_T=ref["final_T"], n_contrib=ref["n_contrib"],
        grad_field=gf,
        **{f"grad_{k}": v for k, v in rb.items() if isinstance(v, np.ndarray)})


def asm_fixture():
    rng = np.random.default_rng(5)
    P, C, H, W, S = 2, 2, 32, 28, 64
    amp = rng.uniform(0, 1, size=(P, C, H, W))
    ph = rng.uniform(0, 2 * np.pi, size=(P, C, H, W))
    fields = (amp * np.exp(1j * ph)).astype(np.complex64)
    wl = np.array([639e-9, 473e-9], np.float32)
    dist = np.array([1.5e-3, -2e-3], np.float32)
    holo = O.multiplane_forward(fields, [float(v) for v in wl], [float(v) for v in dist], PITCH,
                                S, float(S))
    gh = ((rng.normal(size=(C, S, S)) + 1j * rng.normal(size=(C, S, S))) *
          math.sqrt(0.5)).astype(np.complex64)
    adj = O.multiplane_adjoint(gh, H, W, [float(v) for v in wl], [float(v) for v in dist], PITCH,
                               S, float(S))
    return dict(fields=fields, wavelengths=wl, distances=dist,
                setup=np.array([PITCH, S, S], np.float64), hologram=holo.astype(np.complex64),
                grad_hologram=gh, grad_fields=adj.astype(np.complex64))


def geometry_fixture():
    rng = np.random.default_rng(9)
    n = 64
    cam = np.stack([rng.uniform(-1, 1, n), rng.uniform(-1, 1, n), rng.uniform(2, 6, n)], 1)
    cam[:2, 2] = [0.5, 2000.0]  # clipped by near / far
    cam[2, 0] = 30.0            # beyond the Jacobian clamp
    q = rng.normal(size=(n, 4))
    s = np.exp(rng.normal(-3, 0.4, size=(n, 3)))
    th = 0.2
    view = np.array([[math.cos(th), 0, math.sin(th)], [0, 1, 0], [-math.sin(th), 0, math.cos(th)]])
    f32 = lambda a: np.ascontiguousarray(a, np.float32)  # noqa: E731
    cam, q, s, view = f32(cam), f32(q), f32(s), f32(view)
    fx, fy, px, py, W, H = 70.0, 65.0, 32.0, 24.0, 64, 48
    g = O.Gaussians(cam, cam[:, 2].copy(), q, s, np.ones((n, 1), np.float32),
                    np.zeros((n, 1), np.float32), np.ones(n, np.float32),
                    np.ones((n, 1), np.float32))
    c = O.Camera(fx, fy, px, py, view, W, H)
    cov, J, sig, Wr, JW = O.cov2d_forward(g, c)
    pr = O.project(g, c)
    g9, g6, g4, g2 = (f32(rng.normal(size=sh)) for sh in ((n, 3, 3), (n, 2, 3), (n, 2, 2), (n, 2)))
    cq, cs = O.cov3d_backward(g9, q, s)
    jc = O.jacobian_backward(g6, cam, fx, fy, W, H, 1.0, 1000.0)
    c2c, c2q, c2s = O.cov2d_backward(g4, cam, q, s, J, sig, Wr, JW, fx, fy, W, H, 1.0, 1000.0)
    mc = O.means2d_backward(g2, cam, fx, fy, 1.0, 1000.0)
    inv = O.invert_cov2d(cov)
    ginv = O.invert_cov2d_backward(g4, cov)
    return dict(cam=cam, quats=q, scales=s, view=view,
                camera=np.array([fx, fy, px, py, W, H], np.float32),
                cov3d=sig, jacobian=J, cov2d=cov, view_rep=Wr, jw=JW, means2d=pr["means2d"],
                inverse=inv, g9=g9, g6=g6, g4=g4, g2=g2, cov3d_grad_q=cq, cov3d_grad_s=cs,
                jacobian_grad_cam=jc, cov2d_grad_cam=c2c, cov2d_grad_q=c2q, cov2d_grad_s=c2s,
                means2d_grad_cam=mc, inverse_grad=ginv)


FIXTURES = {"raster_small.npz": raster_fixture, "asm_small.npz": asm_fixture,
            "geometry_small.npz": geometry_fixture}


def main():
    for name, fn in FIXTURES.items():
        path = os.path.join(HERE, name)
        np.savez_compressed(path, **fn())
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
