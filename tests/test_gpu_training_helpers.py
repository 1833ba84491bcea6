"""GPU parity of the two training-loop helpers the reference's cov3d_cuda
module exports beside the rasterizer: the fused SSIM map and its image-1
gradient (`fast_ssim`, python_import.py:43-58,449-454; conv.cu:935-1197) and
the sparse Adam step (`sparse_adam_update`, :457-460; spadam.cu), through
the drop-in names, against the oracle's float64 / float32 restatements.

Bars: SSIM map rel-L2 < 1e-5 and gradient rel-L2 < 1e-4 (fp32 window sums
against float64); sparse Adam within 2 float32 ulps-scale (rtol 1e-6)."""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu

SHAPES = [(3, 64, 80), (3, 37, 50), (3, 8, 8), (1, 33, 97), (3, 256, 256)]


def _images(shape, seed):
    rng = np.random.default_rng(seed)
    x = rng.uniform(size=shape).astype(np.float32)
    y = np.clip(x + 0.15 * rng.normal(size=shape), 0, 1).astype(np.float32)
    g = rng.normal(size=shape).astype(np.float32)
    return x, y, g


@pytest.mark.parametrize("shape", SHAPES, ids=["x".join(map(str, s)) for s in SHAPES])
def test_ssim_map_and_gradient(hrf, oracle_mod, shape):
    import torch
    from complex_valued_holographic_radiance_fields_amd import ssim

    print(f"ssim shape={shape}", flush=True)
    x, y, g = _images(shape, sum(shape))
    C1, C2 = 0.01 ** 2, 0.03 ** 2
    tx, ty, tg = (torch.from_numpy(a).cuda() for a in (x, y, g))
    m = ssim.ssim_map(C1, C2, tx, ty)
    gx = ssim.ssim_backward(C1, C2, tx, ty, tg)
    torch.cuda.synchronize()
    assert rel_l2(m.cpu().numpy(), oracle_mod.ssim_map(x, y, C1, C2)) < 1e-5
    assert rel_l2(gx.cpu().numpy(), oracle_mod.ssim_backward(x, y, g, C1, C2)) < 1e-4


def test_fast_ssim_autograd_dropin(hrf, oracle_mod):
    """fast_ssim through the drop-in module: the mean of the map, and the
    autograd gradient of img1 (img2 gets none)."""
    import torch
    from complex_valued_holographic_radiance_fields_amd.cuda_prop.cov3d_cuda import \
        python_import as pi

    x, y, _ = _images((3, 120, 96), 4)
    tx = torch.from_numpy(x).cuda().requires_grad_(True)
    ty = torch.from_numpy(y).cuda().requires_grad_(True)
    val = pi.fast_ssim(tx, ty)
    val.backward()
    torch.cuda.synchronize()
    ref = oracle_mod.ssim_map(x, y, pi.C1, pi.C2)
    assert abs(float(val.detach()) - ref.mean()) < 1e-6
    gref = oracle_mod.ssim_backward(x, y, np.full(x.shape, 1.0 / x.size), pi.C1, pi.C2)
    assert rel_l2(tx.grad.cpu().numpy(), gref) < 1e-4
    assert ty.grad is None
    same = pi.fast_ssim(tx.detach(), tx.detach())
    assert abs(float(same) - 1.0) < 1e-5


@pytest.mark.parametrize("B,N,D,V", [(1, 1000, 3, 400), (3, 5000, 4, 2500), (1, 64, 1, 64)])
def test_sparse_adam_update(hrf, oracle_mod, B, N, D, V):
    import torch
    from complex_valued_holographic_radiance_fields_amd.cuda_prop.cov3d_cuda.python_import \
        import sparse_adam_update

    print(f"sparse adam B={B} N={N} D={D} V={V}", flush=True)
    rng = np.random.default_rng(B * 7 + D)
    p = rng.normal(size=(B, N, D)).astype(np.float32)
    m = (0.1 * rng.normal(size=(B, N, D))).astype(np.float32)
    s = (0.01 * rng.uniform(size=(B, N, D))).astype(np.float32)
    vis = np.sort(rng.choice(N, size=V, replace=False)).astype(np.int64)
    if V > 2:
        vis[1] = N + 5  # out of range: skipped
        vis[2] = -3
    g = rng.normal(size=(B, V, D)).astype(np.float32)
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-15
    tp, tm, ts = (torch.from_numpy(a).cuda() for a in (p, m, s))
    sparse_adam_update(tp, torch.from_numpy(g).cuda(), tm, ts, torch.from_numpy(vis).cuda(), lr,
                       b1, b2, eps)
    torch.cuda.synchronize()
    rp, rm, rs = oracle_mod.sparse_adam_update(p, g, m, s, vis, lr, b1, b2, eps)
    np.testing.assert_allclose(tp.cpu().numpy(), rp, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(tm.cpu().numpy(), rm, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(ts.cpu().numpy(), rs, rtol=1e-6, atol=1e-12)
