"""GPU parity of the fused optimizer step (hrf_grad_norm, hrf_scale_grads,
hrf_adan_step; train.py:319-324, utils/optimizer.py:288-589) against the
oracle and torch.

Bars: parameters and the four state tensors within 1e-6 relative of the
oracle after several steps (the kernel performs the oracle's float32
operations in the same order; the norm is summed in a different order, so
clip coefficients agree to ~1e-7); the gradient norm within 1e-6 of torch's
clip_grad_norm_.  Cases: the reference's seven parameter shapes and learning
rates, odd sizes (vector tails), unaligned views (scalar path), parameters
without gradients, Adan's own max_grad_norm clip, the deferred clip
coefficient, NaN gradients and a state-dict round trip."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# utils/optimizer.py:46-54: (name, learning rate, shape) at lr = 1e-3
GROUPS = [("scales", 0.005, 3), ("phase", 0.0025, 3), ("colours", 0.0025, 3),
          ("means", 1e-3, 3), ("opacity", 0.025, 1), ("plane assignment", 1e-3, 3),
          ("rot", 0.001, 4)]


def _params(n, seed=0):
    import torch

    rng = np.random.default_rng(seed)
    ps = [torch.from_numpy(rng.normal(size=(n, k)).astype(np.float32)).cuda().requires_grad_()
          for _, _, k in GROUPS]
    return ps


def _grads(ps, seed):
    import torch

    rng = np.random.default_rng(seed)
    for p in ps:
        p.grad = torch.from_numpy(rng.normal(scale=0.1, size=tuple(p.shape))
                                  .astype(np.float32)).cuda()


def _oracle_run(oracle_mod, p0, grad_steps, lrs, **kw):
    ps = [p.copy() for p in p0]
    st = [[np.zeros_like(p) for _ in range(4)] for p in p0]
    for k, gs in enumerate(grad_steps, start=1):
        for i in range(len(ps)):
            ps[i], _, *st[i] = oracle_mod.adan_step(ps[i], gs[i], *st[i], lr=lrs[i], step=k, **kw)
    return ps, st


@pytest.mark.parametrize("n", [5003, 2048, 1])
def test_adan_matches_oracle(hrf, oracle_mod, n):
    import torch
    from complex_valued_holographic_radiance_fields_amd.optim import Adan

    ps = _params(n)
    p0 = [p.detach().cpu().numpy().copy() for p in ps]
    opt = Adan([{"params": [p], "lr": lr, "name": name} for p, (name, lr, _) in zip(ps, GROUPS)],
               lr=0, eps=1e-8)
    grads = []
    for k in range(3):
        _grads(ps, seed=10 + k)
        grads.append([p.grad.cpu().numpy().copy() for p in ps])
        opt.step()
    torch.cuda.synchronize()
    print(f"adan n={n}", flush=True)
    exp, est = _oracle_run(oracle_mod, p0, grads, [lr for _, lr, _ in GROUPS])
    for i, p in enumerate(ps):
        np.testing.assert_allclose(p.detach().cpu().numpy(), exp[i], rtol=1e-6, atol=1e-7)
        s = opt.state[p]
        for key, e in zip(("exp_avg", "exp_avg_sq", "exp_avg_diff", "neg_pre_grad"), est[i]):
            np.testing.assert_allclose(s[key].cpu().numpy(), e, rtol=1e-6, atol=1e-10,
                                       err_msg=key)
    assert all(g["step"] == 3 for g in opt.param_groups)


def test_clip_grad_norm_matches_torch_and_oracle(hrf, oracle_mod):
    import torch
    from complex_valued_holographic_radiance_fields_amd import optim

    ps = _params(7001, seed=3)
    _grads(ps, seed=4)
    ref = [p.grad.clone() for p in ps]
    total = optim.clip_grad_norm_(ps, 1.0)
    # torch's own clip on copies of the gradients
    qs = [torch.zeros_like(g, requires_grad=True) for g in ref]
    for q, g in zip(qs, ref):
        q.grad = g.clone()
    t_ref = torch.nn.utils.clip_grad_norm_(qs, 1.0)
    o_total, o_coef, o_scaled = oracle_mod.clip_grad_norm([g.cpu().numpy() for g in ref], 1.0)
    print(f"clip total={float(total):.6f} torch={float(t_ref):.6f}", flush=True)
    assert abs(float(total) - float(t_ref)) <= 1e-6 * float(t_ref)
    assert abs(float(total) - float(o_total)) <= 1e-6 * float(o_total)
    for p, q, e in zip(ps, qs, o_scaled):
        torch.testing.assert_close(p.grad, q.grad, rtol=2e-6, atol=1e-9)
        np.testing.assert_allclose(p.grad.cpu().numpy(), e, rtol=2e-6, atol=1e-9)


def test_deferred_coefficient_equals_clip_then_step(hrf):
    import torch
    from complex_valued_holographic_radiance_fields_amd import optim

    a, b = _params(3001, seed=5), _params(3001, seed=5)
    oa = optim.Adan([{"params": [p], "lr": lr} for p, (_, lr, _) in zip(a, GROUPS)])
    ob = optim.Adan([{"params": [p], "lr": lr} for p, (_, lr, _) in zip(b, GROUPS)])
    for k in range(3):
        _grads(a, seed=20 + k)
        _grads(b, seed=20 + k)
        for p in a + b:
            p.grad.mul_(30.0)  # norms above 1: the clip is active
        optim.clip_grad_norm_(a, 1.0)
        oa.step()
        optim.training_step_update(ob, b, 1.0)
    torch.cuda.synchronize()
    for pa, pb in zip(a, b):
        torch.testing.assert_close(pa, pb, rtol=0, atol=0)
        torch.testing.assert_close(pa.grad, pb.grad, rtol=0, atol=0)


@pytest.mark.parametrize("n", [3, 2047, 2049])
def test_unaligned_views_and_skipped_params(hrf, oracle_mod, n):
    """Views that start one element into their storage take the scalar path;
    a parameter without a gradient is skipped and keeps no state."""
    import torch
    from complex_valued_holographic_radiance_fields_amd.optim import Adan

    rng = np.random.default_rng(n)
    base = torch.from_numpy(rng.normal(size=n + 1).astype(np.float32)).cuda()
    p = base[1:]
    assert p.data_ptr() % 16 != 0
    other = torch.zeros(5, device="cuda")
    opt = Adan([p, other], lr=0.01)
    g = torch.from_numpy(rng.normal(size=n).astype(np.float32)).cuda()
    gbase = torch.zeros(n + 1, device="cuda")
    gbase[1:] = g
    p.grad = gbase[1:]
    p0 = p.detach().cpu().numpy().copy()
    opt.step()
    exp = oracle_mod.adan_step(p0, g.cpu().numpy(), *[np.zeros(n, np.float32)] * 4, lr=0.01,
                               step=1)
    np.testing.assert_allclose(p.detach().cpu().numpy(), exp[0], rtol=1e-6, atol=1e-8)
    assert len(opt.state[other]) == 0


def test_own_max_grad_norm(hrf, oracle_mod):
    """Adan(max_grad_norm=m): clip = clamp(m / (||g|| + eps_last), max=1)
    read back to the host, gradients multiplied by it (optimizer.py:391-409,
    556)."""
    import torch
    from complex_valued_holographic_radiance_fields_amd.optim import Adan

    ps = _params(1001, seed=8)
    _grads(ps, seed=9)
    g = [p.grad.cpu().numpy().copy() for p in ps]
    p0 = [p.detach().cpu().numpy().copy() for p in ps]
    opt = Adan(ps, lr=0.01, max_grad_norm=0.5)
    opt.step()
    total = np.sqrt(sum(float(np.sum(x.astype(np.float64) ** 2)) for x in g))
    clip = min(0.5 / (total + 1e-8), 1.0)
    for i, p in enumerate(ps):
        e = oracle_mod.adan_step(p0[i], g[i], *[np.zeros_like(g[i])] * 4, lr=0.01, step=1,
                                 clip=clip)
        np.testing.assert_allclose(p.detach().cpu().numpy(), e[0], rtol=1e-5, atol=1e-8)
        np.testing.assert_allclose(p.grad.cpu().numpy(), e[1], rtol=1e-5, atol=1e-9)
    torch.cuda.synchronize()


def test_nan_gradient_propagates_like_the_oracle(hrf, oracle_mod):
    import torch
    from complex_valued_holographic_radiance_fields_amd import optim

    p = torch.ones(9, device="cuda", requires_grad=True)
    g = torch.linspace(-1, 1, 9, device="cuda")
    g[4] = float("nan")
    p.grad = g.clone()
    total, coef = optim.grad_norm_clip_coef([p], 1.0)
    assert bool(torch.isnan(total)) and bool(torch.isnan(coef))
    opt = optim.Adan([p], lr=0.01)
    opt.step()
    e = oracle_mod.adan_step(np.ones(9, np.float32), g.cpu().numpy(),
                             *[np.zeros(9, np.float32)] * 4, lr=0.01, step=1)
    np.testing.assert_array_equal(np.isnan(p.detach().cpu().numpy()), np.isnan(e[0]))


def test_state_dict_round_trip(hrf):
    """Saving and reloading the optimizer mid-run continues exactly."""
    import torch
    from complex_valued_holographic_radiance_fields_amd.optim import Adan

    a, b = _params(777, seed=11), _params(777, seed=11)
    oa = Adan([{"params": [p], "lr": lr} for p, (_, lr, _) in zip(a, GROUPS)])
    ob = Adan([{"params": [p], "lr": lr} for p, (_, lr, _) in zip(b, GROUPS)])
    for k in range(2):
        _grads(a, seed=30 + k)
        _grads(b, seed=30 + k)
        oa.step()
        ob.step()
    sd = ob.state_dict()
    ob2 = Adan([{"params": [p], "lr": lr} for p, (_, lr, _) in zip(b, GROUPS)])
    ob2.load_state_dict(sd)
    _grads(a, seed=40)
    _grads(b, seed=40)
    oa.step()
    ob2.step()
    torch.cuda.synchronize()
    for pa, pb in zip(a, b):
        torch.testing.assert_close(pa, pb, rtol=0, atol=0)
