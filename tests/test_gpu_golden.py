"""The HIP library against the committed golden fixtures (tests/golden),
through the same C ABI entry points as the other GPU tests.  Bars: index
outputs bit-exact; fields and gradients rel-L2 < 1e-4; geometry operators
forward bit-exact, backward rel-L2 < 1e-6."""
import os

import numpy as np
import pytest

from conftest import REPO, rel_l2

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(REPO, "tests", "golden")


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_raster_golden(hrf):
    import torch
    from complex_valued_holographic_radiance_fields_amd import rasterizer

    d = np.load(os.path.join(GOLDEN, "raster_small.npz"))
    fx, fy, px, py = (float(v) for v in d["camera"])
    W, H = (int(v) for v in d["img"])
    args = [_t(d[k]) for k in ("cam_means", "z", "quats", "scales", "colours", "phase", "opac",
                               "pprobs")]
    field, (fT, nc, pl, ranges, vis) = rasterizer.forward(*args, fx, fy, px, py, _t(d["view"]),
                                                          (W, H), (16, 16), 1.0, 1000.0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(pl.cpu().numpy(), d["point_list"])
    np.testing.assert_array_equal(ranges.cpu().numpy(), d["ranges"])
    np.testing.assert_array_equal(vis.cpu().numpy(), d["visible"])
    assert rel_l2(field.cpu().numpy(), d["field"]) < 1e-4
    assert rel_l2(fT.cpu().numpy(), d["final_T"]) < 1e-4
    assert np.mean(nc.cpu().numpy() != d["n_contrib"]) < 1e-3
    grads = rasterizer.backward(_t(d["grad_field"]), *args, fx, fy, px, py, _t(d["view"]),
                                (W, H), (16, 16), _t(d["final_T"]), _t(d["n_contrib"]),
                                _t(d["point_list"]), _t(d["ranges"]), 1.0, 1000.0)
    names = ["cam", "z", "quats", "scales", "colours", "phase", "opac", "plane"]
    for name, gg in zip(names, grads):
        err = rel_l2(gg.cpu().numpy(), d[f"grad_{name}"])
        assert err < 1e-4, (name, err)


def test_asm_golden(hrf):
    from complex_valued_holographic_radiance_fields_amd import propagation

    d = np.load(os.path.join(GOLDEN, "asm_small.npz"))
    pitch, S = float(d["setup"][0]), int(d["setup"][1])
    wl = [float(v) for v in d["wavelengths"]]
    dist = [float(v) for v in d["distances"]]
    P, C, H, W = d["fields"].shape
    holo = propagation.multiplane(_t(d["fields"]), wl, pitch, dist, (S, S), float(S))
    assert rel_l2(holo.cpu().numpy(), d["hologram"]) < 1e-4
    adj = propagation.multiplane_adjoint(_t(d["grad_hologram"]), (H, W), wl, pitch, dist, (S, S),
                                         float(S))
    assert rel_l2(adj.cpu().numpy(), d["grad_fields"]) < 1e-4


def test_geometry_golden(hrf):
    from complex_valued_holographic_radiance_fields_amd import geometry as G

    d = np.load(os.path.join(GOLDEN, "geometry_small.npz"))
    fx, fy, px, py, W, H = (float(v) for v in d["camera"])
    W, H = int(W), int(H)
    cam, q, s, view = (_t(d[k]) for k in ("cam", "quats", "scales", "view"))
    np.testing.assert_array_equal(G.cov3d_forward(q, s).cpu().numpy(), d["cov3d"])
    np.testing.assert_array_equal(
        G.means2d_forward(cam, fx, fy, px, py, 1.0, 1000.0).cpu().numpy(), d["means2d"])
    out = G.cov2d_forward(cam, q, s, view, fx, fy, W, H, 1.0, 1000.0)
    for got, key in zip(out, ("cov2d", "jacobian", "cov3d", "view_rep", "jw")):
        np.testing.assert_array_equal(got.cpu().numpy(), d[key])
    np.testing.assert_array_equal(G.invert_cov2d_forward(_t(d["cov2d"])).cpu().numpy(),
                                  d["inverse"])
    gq, gs = G.cov3d_backward(_t(d["g9"]), q, s)
    assert rel_l2(gq.cpu().numpy(), d["cov3d_grad_q"]) < 1e-6
    assert rel_l2(gs.cpu().numpy(), d["cov3d_grad_s"]) < 1e-6
    gj = G.jacobian_backward(_t(d["g6"]), cam, fx, fy, W, H, 1.0, 1000.0)
    assert rel_l2(gj.cpu().numpy(), d["jacobian_grad_cam"]) < 1e-6
    gc, gq2, gs2 = G.cov2d_backward(_t(d["g4"]), cam, q, s, view, _t(d["jacobian"]),
                                    _t(d["cov3d"]), _t(d["view_rep"]), _t(d["jw"]), fx, fy, W, H,
                                    1.0, 1000.0)
    for got, key in ((gc, "cov2d_grad_cam"), (gq2, "cov2d_grad_q"), (gs2, "cov2d_grad_s")):
        assert rel_l2(got.cpu().numpy(), d[key]) < 1e-6
    gm = G.means2d_backward(_t(d["g2"]), cam, fx, fy, px, py, 1.0, 1000.0)
    assert rel_l2(gm.cpu().numpy(), d["means2d_grad_cam"]) < 1e-6
    gi = G.invert_cov2d_backward(_t(d["g4"]), _t(d["cov2d"]))
    assert rel_l2(gi.cpu().numpy(), d["inverse_grad"]) < 1e-6
