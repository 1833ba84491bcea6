"""GPU parity of the standalone geometry operators (compute_cov3d / jacobian /
cov2d / means2d / invert_cov2d, forward and backward) against the oracle,
through the C ABI and through the compat autograd operators.

Bars: forward outputs bit-exact (same arithmetic order, no contraction);
backward rel-L2 < 1e-6.  Inputs include clipped points (outside near/far)
and points beyond the Jacobian clamp."""
import math

import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu

FX, FY, PX, PY, W, H, NEAR, FAR = 90.0, 85.0, 40.0, 30.0, 80, 60, 1.0, 1000.0


def _inputs(n=4000, seed=3):
    rng = np.random.default_rng(seed)
    cam = np.stack([rng.uniform(-2, 2, n), rng.uniform(-2, 2, n), rng.uniform(0.5, 8, n)], 1)
    cam[:5, 2] = [0.2, 1.0, 1000.0, 1500.0, -3.0]  # clipped by near/far
    cam[5:10, 0] = 50.0  # beyond the clamp
    q = rng.normal(size=(n, 4))
    s = np.exp(rng.normal(-3, 0.5, size=(n, 3)))
    th = 0.3
    view = np.array([[math.cos(th), 0, math.sin(th)], [0, 1, 0], [-math.sin(th), 0, math.cos(th)]])
    f32 = lambda a: np.ascontiguousarray(a, np.float32)  # noqa: E731
    return f32(cam), f32(q), f32(s), f32(view)


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _oracle_gaussians(oracle_mod, cam, q, s, view):
    n = cam.shape[0]
    g = oracle_mod.Gaussians(cam, cam[:, 2].copy(), q, s, np.ones((n, 1), np.float32),
                             np.zeros((n, 1), np.float32), np.ones(n, np.float32),
                             np.ones((n, 1), np.float32))
    c = oracle_mod.Camera(FX, FY, PX, PY, view, W, H)
    return g, c


def test_forward_ops_bit_exact(hrf, oracle_mod):
    from complex_valued_holographic_radiance_fields_amd import geometry as G

    cam, q, s, view = _inputs()
    g, c = _oracle_gaussians(oracle_mod, cam, q, s, view)
    cov, J, sig, Wr, JW = oracle_mod.cov2d_forward(g, c)
    pr = oracle_mod.project(g, c)
    print(f"geometry forward n={cam.shape[0]}", flush=True)
    np.testing.assert_array_equal(G.cov3d_forward(_t(q), _t(s)).cpu().numpy(), sig)
    np.testing.assert_array_equal(
        G.jacobian_forward(_t(cam), FX, FY, W, H, NEAR, FAR).cpu().numpy(), J)
    np.testing.assert_array_equal(
        G.means2d_forward(_t(cam), FX, FY, PX, PY, NEAR, FAR).cpu().numpy(), pr["means2d"])
    out = G.cov2d_forward(_t(cam), _t(q), _t(s), _t(view), FX, FY, W, H, NEAR, FAR)
    for got, exp in zip(out, (cov, J, sig, Wr, JW)):
        np.testing.assert_array_equal(got.cpu().numpy(), exp)
    inv = G.invert_cov2d_forward(_t(cov)).cpu().numpy()
    np.testing.assert_array_equal(inv, oracle_mod.invert_cov2d(cov))


def test_backward_ops_match_oracle(hrf, oracle_mod):
    from complex_valued_holographic_radiance_fields_amd import geometry as G

    cam, q, s, view = _inputs(seed=4)
    n = cam.shape[0]
    g, c = _oracle_gaussians(oracle_mod, cam, q, s, view)
    cov, J, sig, Wr, JW = oracle_mod.cov2d_forward(g, c)
    rng = np.random.default_rng(9)
    r = lambda *sh: rng.normal(size=sh).astype(np.float32)  # noqa: E731
    g9, g6, g4, g2 = r(n, 3, 3), r(n, 2, 3), r(n, 2, 2), r(n, 2)
    print(f"geometry backward n={n}", flush=True)

    gq, gs = G.cov3d_backward(_t(g9), _t(q), _t(s))
    eq, es = oracle_mod.cov3d_backward(g9, q, s)
    assert rel_l2(gq.cpu().numpy(), eq) < 1e-6 and rel_l2(gs.cpu().numpy(), es) < 1e-6

    gj = G.jacobian_backward(_t(g6), _t(cam), FX, FY, W, H, NEAR, FAR).cpu().numpy()
    assert rel_l2(gj, oracle_mod.jacobian_backward(g6, cam, FX, FY, W, H, NEAR, FAR)) < 1e-6

    gc, gq2, gs2 = G.cov2d_backward(_t(g4), _t(cam), _t(q), _t(s), _t(view), _t(J), _t(sig),
                                    _t(Wr), _t(JW), FX, FY, W, H, NEAR, FAR)
    ec, eq2, es2 = oracle_mod.cov2d_backward(g4, cam, q, s, J, sig, Wr, JW, FX, FY, W, H, NEAR,
                                             FAR)
    for got, exp in ((gc, ec), (gq2, eq2), (gs2, es2)):
        assert rel_l2(got.cpu().numpy(), exp) < 1e-6

    gm = G.means2d_backward(_t(g2), _t(cam), FX, FY, PX, PY, NEAR, FAR).cpu().numpy()
    assert rel_l2(gm, oracle_mod.means2d_backward(g2, cam, FX, FY, NEAR, FAR)) < 1e-6

    gi = G.invert_cov2d_backward(_t(g4), _t(cov)).cpu().numpy()
    assert rel_l2(gi, oracle_mod.invert_cov2d_backward(g4, cov)) < 1e-6


def test_compat_autograd_operators(hrf):
    """compute_*_cuda through autograd give the operators' own backward."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import geometry as G
    from complex_valued_holographic_radiance_fields_amd.cuda_prop.cov3d_cuda import \
        python_import as pi

    cam, q, s, view = _inputs(n=500, seed=5)
    tc, tq, ts, tv = (_t(a).requires_grad_(True) for a in (cam, q, s, view))
    cov2d = pi.compute_cov2d_cuda(tc, tq, ts, tv, FX, FY, (W, H), NEAR, FAR)
    inv = pi.invert_cov2d_cuda(cov2d)
    m2 = pi.compute_means2d_cuda(tc, FX, FY, PX, PY, NEAR, FAR)
    sig = pi.compute_cov3d_cuda(tq, ts)
    J = pi.compute_jacobian_cuda(tc, FX, FY, (W, H), NEAR, FAR)
    gen = torch.Generator(device="cuda").manual_seed(6)
    gi, gm, gsg, gj = (torch.randn(x.shape, device="cuda", generator=gen)
                       for x in (inv, m2, sig, J))
    loss = (inv * gi).sum() + (m2 * gm).sum() + (sig * gsg).sum() + (J * gj).sum()
    loss.backward()

    d = lambda x: x.detach()  # noqa: E731
    cov_, J_, sig_, W_, JW_ = G.cov2d_forward(d(tc), d(tq), d(ts), d(tv), FX, FY, W, H, NEAR, FAR)
    gcov = G.invert_cov2d_backward(gi, cov_)
    c1, q1, s1 = G.cov2d_backward(gcov, d(tc), d(tq), d(ts), d(tv), J_, sig_, W_, JW_, FX, FY, W,
                                  H, NEAR, FAR)
    c2 = G.means2d_backward(gm, d(tc), FX, FY, PX, PY, NEAR, FAR)
    q3, s3 = G.cov3d_backward(gsg, d(tq), d(ts))
    c4 = G.jacobian_backward(gj, d(tc), FX, FY, W, H, NEAR, FAR)
    # autograd adds the branches' gradients in its own order: compare within
    # a few ulps of the summands' magnitudes (a sum that cancels keeps the
    # absolute rounding of its largest term)
    def close(got, parts):
        ref = sum(parts)
        scale = sum(p.abs() for p in parts)
        assert bool(((got - ref).abs() <= 1e-6 * scale + 1e-7).all())

    close(tc.grad, [c1, c2, c4])
    close(tq.grad, [q1, q3])
    close(ts.grad, [s1, s3])
    assert tv.grad is None


def test_geometry_shape_errors(hrf):
    import torch
    from complex_valued_holographic_radiance_fields_amd import geometry as G

    with pytest.raises(RuntimeError):
        G.cov3d_forward(torch.zeros((4, 3), device="cuda"), torch.zeros((4, 3), device="cuda"))
    with pytest.raises(RuntimeError):
        G.cov2d_forward(torch.zeros((4, 3), device="cuda"), torch.zeros((4, 4), device="cuda"),
                        torch.zeros((4, 3), device="cuda"), torch.eye(2, device="cuda"), 1.0, 1.0,
                        8, 8, 1.0, 100.0)
