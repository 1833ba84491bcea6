"""GPU parity of the HIP rasterizer against the CPU oracle (C ABI path).

Bars: tile/sort indices (point_list, ranges, K, visible) bit-exact; fields and
the 8 parameter gradients within relative L2 1e-4 (fp32); n_contrib may
differ only where the float exp of the two sides straddles the T < 1e-4
termination test (a tiny fraction of pixels).
"""
import numpy as np
import pytest

from conftest import oracle_inputs, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4

CASES = [
    # name, n, W, H, P, C, layout
    ("tiny", 60, 48, 32, 1, 1, "uniform"),
    ("ragged", 3000, 100, 75, 2, 3, "uniform"),
    ("planes3", 8000, 128, 128, 3, 3, "object"),
    ("c2p4", 5000, 96, 80, 4, 2, "object"),
    # one-tile images: no tile bits to sort (the emitted depth order is the
    # sorted order)
    ("onetile", 40, 16, 16, 2, 3, "object"),
    ("subtile", 30, 8, 12, 1, 3, "object"),
]


def _scene(name, n, W, H, P, C, layout, seed=11):
    from complex_valued_holographic_radiance_fields_amd import scenes

    spec = scenes.small(name, n, W, H, P, C, layout, seed=seed)
    return scenes.generate(spec)


def _run_gpu_forward(sc):
    import torch
    from complex_valued_holographic_radiance_fields_amd import rasterizer, scenes

    t = scenes.to_torch(sc)
    field, info = rasterizer.forward(t["cam_means"], t["z"], t["quats"], t["scales"],
                                     t["colours"], t["phase"], t["opac"], t["pprobs"], sc.fx,
                                     sc.fy, sc.px, sc.py, t["view"],
                                     (sc.spec.width, sc.spec.height), (16, 16), 1.0, 1000.0)
    torch.cuda.synchronize()
    return t, field, info


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_forward_parity(hrf, oracle_mod, case):
    sc = _scene(*case)
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
    print(f"case={case[0]} N={g.n} K={ref['K']}", flush=True)
    assert ref["K"] > 0
    np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    np.testing.assert_array_equal(vis.cpu().numpy(), ref["visible"])
    assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL
    assert rel_l2(fT.cpu().numpy(), ref["final_T"]) < TOL
    mism = np.mean(nc.cpu().numpy() != ref["n_contrib"])
    assert mism < 1e-3, mism


def _shuffle(sc, seed=3):
    perm = np.random.default_rng(seed).permutation(sc.cam_means.shape[0])
    for name in ("cam_means", "z", "quats", "scales", "colours", "phase", "opac", "pprobs"):
        setattr(sc, name, np.ascontiguousarray(getattr(sc, name)[perm]))
    return sc


@pytest.mark.parametrize("case", CASES[1:3], ids=[c[0] for c in CASES[1:3]])
def test_forward_parity_unsorted_depth(hrf, oracle_mod, case):
    """Gaussians not pre-sorted by depth: the device depth sort must run."""
    sc = _shuffle(_scene(*case))
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
    np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL


def _swap(sc, i, j):
    for name in ("cam_means", "z", "quats", "scales", "colours", "phase", "opac", "pprobs"):
        a = getattr(sc, name)
        a[[i, j]] = a[[j, i]]
    return sc


@pytest.mark.parametrize("at", [512, 2999], ids=["block_boundary", "last"])
def test_forward_parity_single_depth_inversion(hrf, oracle_mod, at):
    """Depth order broken at one place only: at the first Gaussian of a
    256-Gaussian projection block (its predecessor is in the previous block)
    or at the last Gaussian of a partial block.  The unsorted-depth flag
    raised by that one block must still start the depth sort."""
    sc = _scene(*CASES[1])
    assert np.all(np.diff(sc.z) >= 0)
    k = at
    while sc.z[k - 1] == sc.z[k]:  # a pair of distinct depths ending at `at` or just before
        k -= 1
    _swap(sc, k - 1, k)
    assert np.sum(np.diff(sc.z) < 0) == 1
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
    print(f"inversion at {k}", flush=True)
    np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    np.testing.assert_array_equal(vis.cpu().numpy(), ref["visible"])
    assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_backward_parity(hrf, oracle_mod, case):
    import torch
    from complex_valued_holographic_radiance_fields_amd import rasterizer

    sc = _scene(*case)
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    rng = np.random.default_rng(5)
    P, C, H, W = g.P, g.C, cam.height, cam.width
    gfield = ((rng.normal(size=(P, C, H, W)) + 1j * rng.normal(size=(P, C, H, W))) *
              np.sqrt(0.5)).astype(np.complex64)
    rb = oracle_mod.rasterize_backward(g, cam, ref, gfield)
    t, _, _ = _run_gpu_forward(sc)
    dev = t["cam_means"].device
    # Feed the oracle's forward state so the backward kernels are compared on
    # identical inputs.
    tt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    grads = rasterizer.backward(tt(gfield), t["cam_means"], t["z"], t["quats"], t["scales"],
                                t["colours"], t["phase"], t["opac"], t["pprobs"], sc.fx, sc.fy,
                                sc.px, sc.py, t["view"], (W, H), (16, 16), tt(ref["final_T"]),
                                tt(ref["n_contrib"]), tt(ref["point_list"]), tt(ref["ranges"]),
                                1.0, 1000.0)
    torch.cuda.synchronize()
    names = ["cam", "z", "quats", "scales", "colours", "phase", "opac", "plane"]
    for name, gg in zip(names, grads):
        got = gg.cpu().numpy()
        exp = rb[name]
        if name == "z":
            assert np.all(got == 0)
            continue
        err = rel_l2(got, exp)
        print(f"{case[0]} grad_{name}: rel_l2={err:.3e}", flush=True)
        assert err < TOL, (name, err)


@pytest.mark.parametrize("opacity", ["few_opaque", "all_opaque"])
def test_parity_alpha_clamp_batches(hrf, oracle_mod, opacity):
    """Batches that stage a member with o w above 0.98 keep the reference's
    alpha = min(0.99, .) clamp; the others run the member loops without it.
    A few Gaussians at opacity 0.999 among 0.73 ones (batches of both
    kinds), or all at 0.999 (every batch clamped, alpha reaching 0.99):
    forward and backward match the oracle."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import rasterizer

    sc = _scene("planes3", 8000, 128, 128, 3, 3, "object")
    if opacity == "all_opaque":
        sc.opac[:] = 0.999
    else:
        rng = np.random.default_rng(3)
        sc.opac[rng.choice(sc.opac.size, 40, replace=False)] = 0.999
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    err_f = rel_l2(field.cpu().numpy(), ref["field"])
    err_t = rel_l2(fT.cpu().numpy(), ref["final_T"])
    mism = (nc.cpu().numpy() != ref["n_contrib"]).mean()
    print(f"{opacity}: field {err_f:.2e} final_T {err_t:.2e} n_contrib mismatch {mism:.1e}",
          flush=True)
    assert err_f < TOL and err_t < TOL and mism < 1e-3
    rng = np.random.default_rng(5)
    P, C, H, W = g.P, g.C, cam.height, cam.width
    gfield = ((rng.normal(size=(P, C, H, W)) + 1j * rng.normal(size=(P, C, H, W))) *
              np.sqrt(0.5)).astype(np.complex64)
    rb = oracle_mod.rasterize_backward(g, cam, ref, gfield)
    dev = t["cam_means"].device
    tt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    grads = rasterizer.backward(tt(gfield), t["cam_means"], t["z"], t["quats"], t["scales"],
                                t["colours"], t["phase"], t["opac"], t["pprobs"], sc.fx, sc.fy,
                                sc.px, sc.py, t["view"], (W, H), (16, 16), tt(ref["final_T"]),
                                tt(ref["n_contrib"]), tt(ref["point_list"]), tt(ref["ranges"]),
                                1.0, 1000.0)
    torch.cuda.synchronize()
    names = ["cam", "z", "quats", "scales", "colours", "phase", "opac", "plane"]
    for name, gg in zip(names, grads):
        if name == "z":
            continue
        err = rel_l2(gg.cpu().numpy(), rb[name])
        print(f"{opacity} grad_{name}: rel_l2={err:.3e}", flush=True)
        assert err < TOL, (name, err)


def test_pair_buffers_sized_from_the_last_call(hrf, oracle_mod):
    """The forward allocates its pair-sized outputs (point_list, visible,
    plane member lists) for the last call's pair count plus an eighth
    before it reads its own count back: a call with fewer pairs than that
    returns views of those buffers, one with more allocates them for its
    count.  Lists and fields match the oracle either way."""
    import dataclasses

    from complex_valued_holographic_radiance_fields_amd import rasterizer, scenes

    base = scenes.small("capacity", 3000, 128, 96, 2, 3, "object", seed=23)
    big = scenes.generate(dataclasses.replace(base, log_scale_mean=-2.5))
    small = scenes.generate(base)
    rasterizer._LAST_PAIRS.clear()

    def check(sc, label):
        g, cam = oracle_inputs(sc)
        ref = oracle_mod.rasterize_forward(g, cam)
        t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
        print(f"{label}: K={ref['K']} storage={pl.untyped_storage().nbytes() // 4}", flush=True)
        assert pl.numel() == ref["K"] and vis.numel() == ref["visible"].size
        np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
        np.testing.assert_array_equal(vis.cpu().numpy(), ref["visible"])
        np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
        assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL
        return ref["K"], pl

    k_big, _ = check(big, "first call")
    k_small, pl = check(small, "fewer pairs")  # views of buffers sized for k_big
    assert k_big > k_small + k_small // 8 + 4096  # the capacity the small call left
    assert pl.untyped_storage().nbytes() // 4 > k_small
    _, pl = check(big, "more pairs")  # beyond k_small's capacity: exact buffers
    assert pl.untyped_storage().nbytes() // 4 == k_big


def test_empty_scene(hrf):
    """All Gaussians behind the near plane: the reference's total_pairs == 0
    path (rasterizer_splat.cu:434-449)."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import rasterizer

    sc = _scene("empty", 50, 40, 40, 2, 3, "uniform")
    sc.z[:] = 0.5
    sc.cam_means[:, 2] = 0.5
    t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
    assert torch.count_nonzero(field).item() == 0
    assert torch.all(fT == 1).item() and torch.all(nc == 0).item()
    assert pl.shape == (1,) and int(pl[0]) == 0
    assert vis.numel() == 0 and torch.all(ranges == 0).item()
    grads = rasterizer.backward(torch.ones_like(field), t["cam_means"], t["z"], t["quats"],
                                t["scales"], t["colours"], t["phase"], t["opac"], t["pprobs"],
                                sc.fx, sc.fy, sc.px, sc.py, t["view"], (40, 40), (16, 16), fT,
                                nc, pl, ranges, 1.0, 1000.0)
    for gg in grads:
        assert torch.count_nonzero(gg).item() == 0


def test_single_gaussian_closed_form(hrf):
    """One isotropic Gaussian centred on a pixel: field = colour*min(.99, o)*e^{i phi}."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import rasterizer

    dev = "cuda"
    f = 100.0
    cam = torch.tensor([[0.0, 0.0, 4.0]], device=dev)
    # pixel (20, 12): mx = fx*(-x/z)+px -> x = -(20-px)*z/fx
    px, py = 16.0, 16.0
    cam[0, 0] = -(20.0 - px) * 4.0 / f
    cam[0, 1] = -(12.0 - py) * 4.0 / f
    z = cam[:, 2].clone()
    q = torch.tensor([[1.0, 0.0, 0.0, 0.0]], device=dev)
    s = torch.full((1, 3), 0.02, device=dev)
    col = torch.tensor([[0.8]], device=dev)
    ph = torch.tensor([[1.1]], device=dev)
    op = torch.tensor([0.7], device=dev)
    pp = torch.ones((1, 1), device=dev)
    view = torch.eye(3, device=dev)
    field, info = rasterizer.forward(cam, z, q, s, col, ph, op, pp, f, f, px, py, view, (32, 32),
                                     (16, 16), 1.0, 1000.0)
    v = field[0, 0, 12, 20].item()
    expect = 0.8 * 0.7 * np.exp(1j * 1.1)
    assert abs(v - expect) < 1e-6
    assert abs(info[0][0, 12, 20].item() - 0.3) < 1e-6
    assert int(info[1][0, 12, 20]) == 1
    # one pair (its 3-pixel radius stays inside tile (1, 0) of the 2 x 2
    # grid): point_list [0], that tile's range [0, 1), the others empty
    np.testing.assert_array_equal(info[2].cpu().numpy(), [0])
    np.testing.assert_array_equal(info[3].cpu().numpy(), [[0, 0], [0, 1], [0, 0], [0, 0]])
    np.testing.assert_array_equal(info[4].cpu().numpy(), [0])


def test_autograd_dropin(hrf):
    """splat_tile_cuda (autograd.Function) returns what Rasterizer returns and
    its backward reproduces Rasterizer.backward.  The two backward runs sum
    per-Gaussian partials with float atomics (as the reference does), so they
    agree to rounding, not bit for bit: compared by relative L2."""
    import torch
    from complex_valued_holographic_radiance_fields_amd.cuda_prop.cov3d_cuda import python_import as pi
    from complex_valued_holographic_radiance_fields_amd import scenes

    sc = _scene("autograd", 2000, 64, 64, 2, 3, "uniform")
    t = scenes.to_torch(sc)
    leaves = [t[k].clone().requires_grad_(True) for k in
              ("cam_means", "z", "quats", "scales", "colours", "phase", "opac", "pprobs")]
    field, vis = pi.splat_tile_cuda(*leaves, sc.fx, sc.fy, sc.px, sc.py, t["view"], (64, 64),
                                    1.0, 1000.0)
    assert vis.dtype == torch.int64
    g = torch.randn(field.shape, dtype=field.dtype, device="cuda",
                    generator=torch.Generator(device="cuda").manual_seed(15))
    (field.real * g.real + field.imag * g.imag).sum().backward()
    ras = pi.Rasterizer()
    out, info = ras.forward(*[x.detach() for x in leaves], sc.fx, sc.fy, sc.px, sc.py, t["view"],
                            (64, 64), (16, 16), 1.0, 1000.0)
    assert torch.equal(out, field.detach())
    grads = ras.backward(g, *[x.detach() for x in leaves], sc.fx, sc.fy, sc.px, sc.py, t["view"],
                         (64, 64), (16, 16), info[0], info[1], info[2], info[3], 1.0, 1000.0)
    for leaf, gr in zip(leaves, grads):
        assert rel_l2(leaf.grad.cpu().numpy(), gr.cpu().numpy()) < 1e-6


def test_bad_channels_raise(hrf):
    import torch
    from complex_valued_holographic_radiance_fields_amd import rasterizer

    n = 4
    d = "cuda"
    with pytest.raises(RuntimeError):
        rasterizer.forward(torch.zeros((n, 3), device=d), torch.ones(n, device=d) * 4,
                           torch.zeros((n, 4), device=d), torch.ones((n, 3), device=d),
                           torch.ones((n, 4), device=d), torch.ones((n, 4), device=d),
                           torch.ones(n, device=d), torch.ones((n, 1), device=d), 10.0, 10.0,
                           8.0, 8.0, torch.eye(3, device=d), (16, 16), (16, 16), 1.0, 1000.0)


def test_count_readback_stream_fallback(hrf, oracle_mod, monkeypatch):
    """The pair / visible counts reach the host through pinned words that
    the scan kernel tags last; with the poll disabled
    (HRF_READBACK_SPIN_US=0) the host takes the stream-synchronisation
    fallback, and both paths give the oracle's lists."""
    sc = _scene(*CASES[1])
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    for spin in ("0", "20000"):
        monkeypatch.setenv("HRF_READBACK_SPIN_US", spin)
        t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
        print(f"spin={spin} K={pl.numel()}", flush=True)
        np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
        np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
        np.testing.assert_array_equal(vis.cpu().numpy(), ref["visible"])
        assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL


def test_concurrent_forwards_on_two_streams(hrf, oracle_mod):
    """Two host threads rasterize different scenes at the same time, each on
    its own stream: the count read-backs use separate pinned slots and every
    result matches the oracle."""
    import threading

    import torch

    scs = [_scene(*CASES[1]), _scene(*CASES[3])]
    refs = []
    for sc in scs:
        g, cam = oracle_inputs(sc)
        refs.append(oracle_mod.rasterize_forward(g, cam))
    errors, outs = [], [[], []]

    def worker(i):
        try:
            st = torch.cuda.Stream()
            with torch.cuda.stream(st):
                for _ in range(4):
                    _, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(scs[i])
                    outs[i].append((pl.cpu().numpy(), ranges.cpu().numpy(),
                                    field.cpu().numpy()))
        except Exception as e:  # reported below
            errors.append(repr(e))

    th = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join(timeout=100)
    print(f"threads done, errors={errors}", flush=True)
    assert not errors
    for i in range(2):
        assert len(outs[i]) == 4
        for pl, ranges, field in outs[i]:
            np.testing.assert_array_equal(ranges, refs[i]["ranges"])
            np.testing.assert_array_equal(pl, refs[i]["point_list"])
            assert rel_l2(field, refs[i]["field"]) < TOL


def test_forward_parity_wide_keys(hrf, oracle_mod):
    """Tile id and gaussian index need more than 32 bits together (16384
    tiles, 270k Gaussians): the binning takes the separate key/value sort
    path instead of the packed one."""
    from complex_valued_holographic_radiance_fields_amd import scenes

    spec = scenes.SceneSpec("wide", 6, 270_000, 2048, 2048, 1, [515e-9], [-2e-3], "uniform",
                            log_scale_mean=-6.0, log_scale_std=0.3)
    sc = scenes.generate(spec)
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    print(f"wide keys: N={g.n} K={ref['K']}", flush=True)
    t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
    np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    np.testing.assert_array_equal(vis.cpu().numpy(), ref["visible"])
    assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL


def test_forward_parity_large_grid_packed(hrf, oracle_mod):
    """A tile grid whose count difference array exceeds the LDS bound (133 x
    133 > 16000 entries) with tile id and index still in one word: the
    packed path unpacks the sorted words for point_list and the ranges."""
    from complex_valued_holographic_radiance_fields_amd import scenes

    spec = scenes.SceneSpec("grid", 7, 6000, 2112, 2112, 1, [515e-9], [-2e-3], "uniform",
                            log_scale_mean=-5.0, log_scale_std=0.3)
    sc = scenes.generate(spec)
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    print(f"large grid: N={g.n} K={ref['K']}", flush=True)
    assert ref["K"] > 1
    t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
    np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL


REGEN_SCENES = {
    # 17689 tiles (15 bits, packed words), few pairs per emission block
    "grid": dict(name="grid", seed=7, n=6000, W=2112, H=2112, P=1, wl=[515e-9], d=[-2e-3],
                 layout="uniform", log_scale_mean=-5.0, log_scale_std=0.3),
    # 1024 tiles (10 bits, packed), several sort tiles of pairs per block
    "mid": dict(name="mid", seed=9, n=60_000, W=512, H=512, P=3, wl=[639e-9, 532e-9, 473e-9],
                d=[-1e-3, 0.0, 1e-3], layout="object", log_scale_mean=-4.0, log_scale_std=0.5),
    # tile and index past 32 bits: separate keys and values
    "wide": dict(name="wide", seed=6, n=270_000, W=2048, H=2048, P=1, wl=[515e-9], d=[-2e-3],
                 layout="uniform", log_scale_mean=-6.0, log_scale_std=0.3),
}


@pytest.mark.parametrize("case", list(REGEN_SCENES))
def test_forward_parity_regenerated_first_pass(hrf, oracle_mod, monkeypatch, case):
    """The fused emission-scatter (the emission only counts the first sort
    pass's digits; that pass regenerates each emission block's pairs and
    scatters them) runs by itself only for sorts of 2^26 pairs or more
    (config 4); HRF_SORT_REGENERATE=1 takes it at these sizes.  The binning
    must equal the oracle's bit for bit, packed and wide keys alike."""
    from complex_valued_holographic_radiance_fields_amd import scenes

    a = REGEN_SCENES[case]
    spec = scenes.SceneSpec(a["name"], a["seed"], a["n"], a["W"], a["H"], a["P"], a["wl"],
                            a["d"], a["layout"], log_scale_mean=a["log_scale_mean"],
                            log_scale_std=a["log_scale_std"])
    sc = scenes.generate(spec)
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    print(f"regenerated first pass, {case}: N={g.n} K={ref['K']}", flush=True)
    monkeypatch.setenv("HRF_SORT_REGENERATE", "1")
    t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
    np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    np.testing.assert_array_equal(vis.cpu().numpy(), ref["visible"])
    assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL


@pytest.mark.parametrize("case", ["grid", "mid"])
def test_forward_parity_emission_histogram(hrf, oracle_mod, monkeypatch, case):
    """The pair emission taking the first sort pass's histogram over groups
    of its blocks (the pass's partitions, partial tiles at their edges) and
    storing the pairs for that pass: chosen by itself only for sorts of 2^26
    pairs or more whose emission blocks hold few pairs;
    HRF_SORT_REGENERATE=2 takes it at these sizes.  Binning bit-exact."""
    from complex_valued_holographic_radiance_fields_amd import scenes

    a = REGEN_SCENES[case]
    spec = scenes.SceneSpec(a["name"], a["seed"], a["n"], a["W"], a["H"], a["P"], a["wl"],
                            a["d"], a["layout"], log_scale_mean=a["log_scale_mean"],
                            log_scale_std=a["log_scale_std"])
    sc = scenes.generate(spec)
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    print(f"emission histogram, {case}: N={g.n} K={ref['K']}", flush=True)
    monkeypatch.setenv("HRF_SORT_REGENERATE", "2")
    t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
    np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    np.testing.assert_array_equal(vis.cpu().numpy(), ref["visible"])
    assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL


def _plane_list_scene(case):
    import dataclasses

    from complex_valued_holographic_radiance_fields_amd import scenes

    if case == "dense":
        # Opaque, large Gaussians: ~40% of the pixels reach T < 1e-4, so the
        # forward stops early and the plane lists end before the tile lists.
        spec = dataclasses.replace(scenes.small("dense", 4000, 48, 48, 2, 3, "uniform", seed=21),
                                   log_scale_mean=-2.5)
        sc = scenes.generate(spec)
        sc.opac[:] = 0.95
        return sc
    sc = _scene("planes3", 8000, 128, 128, 3, 3, "object")
    if case == "soft":
        # Soft plane weights: Gaussians in several planes, some weights at
        # zero or below the 1e-6 cutoff.
        rng = np.random.default_rng(8)
        w = rng.uniform(0, 1, size=sc.pprobs.shape).astype(np.float32)
        w[rng.uniform(size=w.shape) < 0.3] = 0.0
        w[rng.uniform(size=w.shape) < 0.05] = 5e-7
        sc.pprobs[:] = w
    return sc


@pytest.mark.parametrize("case", ["onehot", "soft", "dense"])
def test_backward_with_plane_lists(hrf, oracle_mod, case):
    """The forward's plane member lists (kept for the backward): each
    (tile, plane) list is exactly that plane's members of the tile list, in
    list order, cut after the last batch the forward composited (never before
    any pixel's n_contrib); the block order the backward writes into the
    same buffer is a permutation sorted by list length; the backward walking
    them matches the oracle's
    backward on the same forward state and the backward that filters the tile
    lists itself (both sum float atomics, so to rounding: rel-L2 < 1e-6)."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import rasterizer, scenes

    sc = _plane_list_scene(case)
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    t = scenes.to_torch(sc)
    W, H = sc.spec.width, sc.spec.height
    args = (t["cam_means"], t["z"], t["quats"], t["scales"], t["colours"], t["phase"], t["opac"],
            t["pprobs"], sc.fx, sc.fy, sc.px, sc.py, t["view"])
    field, info, geom = rasterizer.forward(*args, (W, H), (16, 16), 1.0, 1000.0,
                                           keep_geometry=True)
    fT, nc, pl, ranges, _ = info
    torch.cuda.synchronize()
    assert geom.plane_lists is not None
    P, K = g.P, int(pl.numel())
    print(f"case={case} N={g.n} K={K} P={P}", flush=True)
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    if case == "dense":
        assert float((fT < 1e-4).float().mean()) > 0.2

    # Plane lists: P*K (gaussian, position) pairs, then, from the next
    # 256-byte boundary, T*P counts.
    buf = geom.plane_lists.cpu().numpy()
    ntiles = ranges.shape[0]
    ent = buf[:P * K * 8].view(np.int32).reshape(P, K, 2)
    # entry: (gaussian, list position | quadrant mask << 28)
    epos = (ent[..., 1].view(np.uint32) & 0x0FFFFFFF).astype(np.int64)
    emask = ent[..., 1].view(np.uint32) >> 28
    c0 = (P * K * 8 + 255) // 256 * 256
    cnt = buf[c0:c0 + ntiles * P * 4].view(np.int32).reshape(ntiles, P)
    o0 = (c0 + ntiles * P * 4 + 255) // 256 * 256
    pl_np, r_np, nc_np = pl.cpu().numpy(), ranges.cpu().numpy(), nc.cpu().numpy()
    member = g.pprobs >= np.float32(1e-6)
    # float64 alpha of a Gaussian over a tile's pixel centres
    pr = ref["proj"]
    m2, cov = pr["means2d"].astype(np.float64), pr["cov2d"].astype(np.float64)
    det = cov[:, 0] * cov[:, 3] - cov[:, 1] * cov[:, 2]
    cxx, cxy, czz = cov[:, 3] / det, -cov[:, 1] / det, cov[:, 0] / det
    gx = (W + 15) // 16
    # quadrant w of the tile: pixels (w & 1) * 8 .. +8 across, (w >> 1) * 8 .. +8 down
    quad_of = ((np.repeat(np.arange(16), 16) >= 8) * 2 + (np.tile(np.arange(16), 16) >= 8))

    def alpha_tile(gg, p, px, py):
        dx = m2[gg, 0][:, None] - px[None, :]
        dy = m2[gg, 1][:, None] - py[None, :]
        q = cxx[gg][:, None] * dx * dx + 2 * cxy[gg][:, None] * dx * dy \
            + czz[gg][:, None] * dy * dy
        ow = g.opac[gg].astype(np.float64) * g.pprobs[gg, p]
        return ow[:, None] * np.exp(-0.5 * q)

    truncated = invisible = faint = listed = 0
    for tile in range(ntiles):
        r0, r1 = r_np[tile]
        ty, tx = divmod(tile, gx)
        px = np.tile(np.arange(16), 16) + tx * 16.0
        py = np.repeat(np.arange(16), 16) + ty * 16.0
        for p in range(P):
            tile_nc = nc_np[p, ty * 16:(ty + 1) * 16, tx * 16:(tx + 1) * 16]
            ks = np.nonzero(member[pl_np[r0:r1], p])[0]
            c = int(cnt[tile, p])
            assert 0 <= c <= len(ks)
            got, gpos, gmask = ent[p, r0:r0 + c], epos[p, r0:r0 + c], emask[p, r0:r0 + c]
            # the list: plane members in list order ...
            assert np.all(np.diff(gpos) > 0) and np.all(np.isin(gpos, ks))
            np.testing.assert_array_equal(got[:, 0], pl_np[r0 + gpos])
            # ... each with the quadrants where it reaches alpha >= 1/255
            # (the kernel's test has a margin of ~1% in alpha on the inside)
            if c:
                gg = pl_np[r0 + gpos]
                aq = alpha_tile(gg, p, px, py)
                amax = np.stack([aq[:, quad_of == w].max(1) for w in range(4)], 1)
                # over the box spanned by the quadrant's pixel centres
                abox = np.stack([_alpha_box_max(m2[gg], cxx[gg], cxy[gg], czz[gg],
                                                g.opac[gg].astype(np.float64) * g.pprobs[gg, p],
                                                tx * 16 + (w & 1) * 8, ty * 16 + (w >> 1) * 8, 7.0)
                                 for w in range(4)], 1)
                bits = (gmask[:, None] >> np.arange(4)) & 1
                assert np.all(gmask != 0)
                assert np.all(abox[bits == 1] >= 0.98 / 255), (tile, p)
                assert np.all(amax[bits == 0] < (1 + 1e-5) / 255), (tile, p)
                listed += c
            # ... and every member it leaves out lies beyond every pixel's
            # n_contrib, has alpha < 2^-25 at every pixel of the tile (culled
            # by the forward as without effect) or alpha < 1/255 at every
            # pixel (nothing for the backward)
            missing = np.setdiff1d(ks, gpos)
            inner = missing[missing < tile_nc.max()]
            if len(inner):
                alpha = alpha_tile(pl_np[r0 + inner], p, px, py).max(1)
                assert np.all(alpha < (1 + 1e-5) / 255), (tile, p, alpha.max())
                invisible += int(np.sum(alpha < 2.0 ** -25))
                faint += int(np.sum(alpha >= 2.0 ** -25))
            if np.any(missing >= tile_nc.max()):
                truncated += 1
    print(f"plane lists: {listed} listed, {truncated} cut short, {invisible} invisible and "
          f"{faint} faint members left out", flush=True)
    if case == "dense":
        assert truncated > 0

    rng = np.random.default_rng(6)
    gf = ((rng.normal(size=(P, g.C, H, W)) + 1j * rng.normal(size=(P, g.C, H, W))) *
          np.sqrt(0.5)).astype(np.complex64)
    gft = torch.from_numpy(gf).cuda()
    with_lists = rasterizer.backward(gft, *args, (W, H), (16, 16), fT, nc, pl, ranges, 1.0, 1000.0,
                                     geometry=geom)
    filtered = rasterizer.backward(gft, *args, (W, H), (16, 16), fT, nc, pl, ranges, 1.0, 1000.0)
    # The block order the backward wrote after the counts: a permutation of
    # the (tile, plane) ids, counts non-increasing at the granularity of 8
    # buckets per octave.
    torch.cuda.synchronize()
    order = geom.plane_lists.cpu().numpy()[o0:o0 + ntiles * P * 4].view(np.int32)
    np.testing.assert_array_equal(np.sort(order), np.arange(ntiles * P))
    v = np.maximum(cnt.reshape(-1)[order].astype(np.int64), 0) + 1
    e = np.floor(np.log2(v)).astype(np.int64)
    mant = np.where(e >= 3, v >> np.maximum(e - 3, 0), v << np.maximum(3 - e, 0)) & 7
    assert np.all(np.diff(e * 8 + mant) <= 0)
    state = dict(ref, final_T=fT.cpu().numpy(), n_contrib=nc_np, point_list=pl_np, ranges=r_np)
    rb = oracle_mod.rasterize_backward(g, cam, state, gf)
    names = ["cam", "z", "quats", "scales", "colours", "phase", "opac", "plane"]
    for name, a, b in zip(names, with_lists, filtered):
        a, b = a.cpu().numpy(), b.cpu().numpy()
        if name == "z":
            assert np.all(a == 0)
            continue
        assert rel_l2(a, b) < 1e-6, name
        err = rel_l2(a, rb[name])
        print(f"{case} grad_{name}: rel_l2={err:.3e}", flush=True)
        assert err < TOL, (name, err)


def _alpha_box_max(m2, cxx, cxy, czz, ow, x0, y0, ext):
    """float64 max of o w exp(-q/2) over the box [x0, x0+ext] x [y0, y0+ext]
    (q = d^T A d, d = mean - point; A positive definite): the minimum of q
    is 0 with the mean inside, else on the boundary, where each edge is a
    1-D convex quadratic minimised by clamping its vertex."""
    mx, my = m2[:, 0], m2[:, 1]
    inside = (mx >= x0) & (mx <= x0 + ext) & (my >= y0) & (my <= y0 + ext)
    best = np.full(len(mx), np.inf)
    for fixed_x in (True, False):
        for edge in (0.0, ext):
            if fixed_x:
                dx = mx - (x0 + edge)
                # q(dy) = czz dy^2 + 2 cxy dx dy + cxx dx^2, dy = my - y, y in [y0, y0+ext]
                dy = np.clip(-cxy * dx / czz, my - (y0 + ext), my - y0)
            else:
                dy = my - (y0 + edge)
                dx = np.clip(-cxy * dy / cxx, mx - (x0 + ext), mx - x0)
            best = np.minimum(best, cxx * dx * dx + 2 * cxy * dx * dy + czz * dy * dy)
    q = np.where(inside, 0.0, best)
    return ow * np.exp(-0.5 * q)


@pytest.mark.parametrize("W,H", [(16, 16), (8, 12)])
def test_one_tile_frame_with_plane_lists(hrf, oracle_mod, W, H):
    """Images that fit one tile on the benchmark's path (forward records and
    plane member lists kept, backward reusing them): lists, field and the
    8 gradients against the oracle."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import rasterizer

    sc = _scene("onetile_pl", 60, W, H, 3, 3, "object", seed=4)
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    assert ref["K"] > 1
    t = scenes_torch(sc)
    field, info, geom = rasterizer.forward(t["cam_means"], t["z"], t["quats"], t["scales"],
                                           t["colours"], t["phase"], t["opac"], t["pprobs"],
                                           sc.fx, sc.fy, sc.px, sc.py, t["view"], (W, H),
                                           (16, 16), 1.0, 1000.0, keep_geometry=True)
    fT, nc, pl, ranges, vis = info
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
    assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL
    rng = np.random.default_rng(8)
    gf = (rng.normal(size=field.shape) + 1j * rng.normal(size=field.shape)).astype(np.complex64)
    grads = rasterizer.backward(torch.from_numpy(gf).cuda(), t["cam_means"], t["z"], t["quats"],
                                t["scales"], t["colours"], t["phase"], t["opac"], t["pprobs"],
                                sc.fx, sc.fy, sc.px, sc.py, t["view"], (W, H), (16, 16), fT, nc,
                                pl, ranges, 1.0, 1000.0, geometry=geom)
    torch.cuda.synchronize()
    rb = oracle_mod.rasterize_backward(g, cam, ref, gf)
    for name, gg in zip(["cam", "z", "quats", "scales", "colours", "phase", "opac", "plane"],
                        grads):
        assert rel_l2(gg.cpu().numpy(), rb[name]) < TOL, name


def scenes_torch(sc):
    from complex_valued_holographic_radiance_fields_amd import scenes

    return scenes.to_torch(sc)


def _nan_close(got, exp, tol):
    """NaN in the same places, the finite entries within rel-L2 tol."""
    np.testing.assert_array_equal(np.isnan(got), np.isnan(exp))
    fin = ~np.isnan(exp)
    assert rel_l2(np.where(fin, got, 0), np.where(fin, exp, 0)) < tol


def test_degenerate_gaussians_are_culled(hrf, oracle_mod):
    """A zero quaternion (its normalisation divides by zero), a NaN or
    infinite scale and a NaN quaternion make the covariance and so the
    radius NaN; a NaN camera-space x makes the 2-D mean NaN (the Jacobian's
    clamp keeps the covariance finite).  Such a Gaussian is culled (it
    joins no tile list), on the GPU as in the oracle, and the rest of the
    frame matches.  Their gradients are what the geometry backward makes of them
    (NaN, as the reference's chain rule through NaN gives)."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import rasterizer

    sc = _scene(*CASES[1])
    bad = [5, 17, 33, 260, 1200, 2999]
    sc.quats[5] = 0.0
    sc.scales[17, 1] = np.nan
    sc.scales[33, 0] = np.inf
    sc.quats[260, 2] = np.nan
    sc.cam_means[1200, 0] = np.nan
    sc.scales[2999] = np.inf
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    assert np.all(ref["tiles"][bad] == 0)
    t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
    pl_h = pl.cpu().numpy()
    assert not np.isin(pl_h, bad).any()
    np.testing.assert_array_equal(pl_h, ref["point_list"])
    np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
    np.testing.assert_array_equal(vis.cpu().numpy(), ref["visible"])
    f_h = field.cpu().numpy()
    assert np.isfinite(f_h).all()
    assert rel_l2(f_h, ref["field"]) < TOL
    rng = np.random.default_rng(9)
    gf = (rng.normal(size=f_h.shape) + 1j * rng.normal(size=f_h.shape)).astype(np.complex64)
    rb = oracle_mod.rasterize_backward(g, cam, ref, gf)
    tt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    grads = rasterizer.backward(tt(gf), t["cam_means"], t["z"], t["quats"], t["scales"],
                                t["colours"], t["phase"], t["opac"], t["pprobs"], sc.fx, sc.fy,
                                sc.px, sc.py, t["view"], (cam.width, cam.height), (16, 16),
                                tt(ref["final_T"]), tt(ref["n_contrib"]), tt(ref["point_list"]),
                                tt(ref["ranges"]), 1.0, 1000.0)
    torch.cuda.synchronize()
    good = np.setdiff1d(np.arange(g.n), bad)
    for name, gg in zip(["cam", "z", "quats", "scales", "colours", "phase", "opac", "plane"],
                        grads):
        got = gg.cpu().numpy()
        if name == "z":
            assert not got.any()
            continue
        print(f"degenerate grad_{name}: NaN rows gpu {np.unique(np.nonzero(np.isnan(got))[0])} "
              f"oracle {np.unique(np.nonzero(np.isnan(rb[name]))[0])}", flush=True)
        assert rel_l2(got[good], rb[name][good]) < TOL, name
        _nan_close(got, rb[name], TOL)


def test_render_rejects_counts_other_than_prepared(hrf):
    """hrf_raster_forward_render given counts other than the ones prepare
    returned for the workspace: HRF_ERR_INVALID before any launch; the right
    counts then work."""
    import ctypes

    import torch
    from complex_valued_holographic_radiance_fields_amd import _lib

    sc = _scene(*CASES[1])
    t = scenes_torch(sc)
    lib = _lib.load()
    dev = t["cam_means"].device
    n, C, P = sc.cam_means.shape[0], sc.colours.shape[1], sc.pprobs.shape[1]
    W, H = sc.spec.width, sc.spec.height
    g = _lib.HrfGaussians(t["cam_means"].data_ptr(), t["z"].data_ptr(), t["quats"].data_ptr(),
                          t["scales"].data_ptr(), t["colours"].data_ptr(), t["phase"].data_ptr(),
                          t["opac"].data_ptr(), t["pprobs"].data_ptr(), n, C, P)
    c = _lib.HrfCamera(sc.fx, sc.fy, sc.px, sc.py, t["view"].data_ptr(), W, H, 1.0, 1000.0)
    stream = _lib.stream_ptr(dev)
    gb = lib.hrf_raster_geom_workspace_size(n, C, P)
    gws = torch.empty(gb, dtype=torch.uint8, device=dev)
    K, V = ctypes.c_int64(0), ctypes.c_int64(0)
    _lib.check(lib.hrf_raster_forward_prepare(ctypes.byref(g), ctypes.byref(c), gws.data_ptr(),
                                              gb, stream, ctypes.byref(K), ctypes.byref(V)))
    K, V = K.value, V.value
    assert K > 10
    bb = lib.hrf_raster_binning_workspace_size(K + 5, W, H)
    bws = torch.empty(bb, dtype=torch.uint8, device=dev)
    field = torch.empty((P, C, H, W), dtype=torch.complex64, device=dev)
    fT = torch.empty((P, H, W), device=dev)
    nc = torch.empty((P, H, W), dtype=torch.int32, device=dev)
    pl = torch.empty(K + 5, dtype=torch.int32, device=dev)
    rg = torch.empty((((W + 15) // 16) * ((H + 15) // 16), 2), dtype=torch.int32, device=dev)
    vis = torch.empty(V + 5, dtype=torch.int64, device=dev)

    def render(k, v):
        return lib.hrf_raster_forward_render(ctypes.byref(g), ctypes.byref(c), gws.data_ptr(),
                                             gb, bws.data_ptr(), bb, k, v, field.data_ptr(),
                                             fT.data_ptr(), nc.data_ptr(), pl.data_ptr(),
                                             rg.data_ptr(), vis.data_ptr(), None, 0, stream)

    for k, v in ((K - 1, V), (K + 1, V), (K, V - 1), (K, V + 1)):
        assert render(k, v) == 1, (k, v)
        err = lib.hrf_last_error()
        # V + 1 can exceed N (every Gaussian visible): the count check fires first
        assert b"differ" in err or (v > n and b"invalid visible count" in err), err
    assert render(K, V) == 0
    torch.cuda.synchronize()
    ref, _, (_, _, pl_ref, rg_ref, vis_ref) = _run_gpu_forward(sc)
    assert torch.equal(pl[:K], pl_ref) and torch.equal(rg, rg_ref)
    assert torch.equal(vis[:V], vis_ref)


def test_forward_parity_dense_terminations(hrf, oracle_mod):
    """Opaque, large Gaussians (the "dense" plane-list scene): about 40% of
    the pixels stop at T < 1e-4, many in the middle of a 256-entry batch or
    of an 8-member group of the member loop.  The field, final_T and
    n_contrib of terminated pixels (the list position of the member that
    took T below 1e-4) match the oracle."""
    sc = _plane_list_scene("dense")
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    t, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
    fT_h, nc_h = fT.cpu().numpy(), nc.cpu().numpy()
    term = ref["final_T"] < 1e-4
    print(f"dense: K={ref['K']} terminated {term.mean():.2f}", flush=True)
    assert term.mean() > 0.2
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL
    assert rel_l2(fT_h, ref["final_T"]) < TOL
    mism = nc_h != ref["n_contrib"]
    assert mism.mean() < 1e-3, (mism.mean(), np.argwhere(mism)[:5])
    # where the two sides terminate at the same member, n_contrib is equal
    both = term & (fT_h < 1e-4)
    assert np.mean(nc_h[both] != ref["n_contrib"][both]) < 1e-3


def test_allocation_failure_then_recovery(hrf, oracle_mod):
    """An allocation that cannot be satisfied (a 200000 x 200000 image: the
    (P,C,H,W) field alone would be petabytes) raises RuntimeError at the
    boundary before any kernel runs, as the reference's buffer resizes do
    (rasterizer_splat.cu:217-222); the next, ordinary frame on the same
    device is still exact."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import rasterizer, scenes

    sc = _scene("small", 400, 64, 48, 2, 3, "object")
    t = scenes.to_torch(sc)
    print("allocation failure: 200000 x 200000 request", flush=True)
    with pytest.raises(RuntimeError):
        rasterizer.forward(t["cam_means"], t["z"], t["quats"], t["scales"], t["colours"],
                           t["phase"], t["opac"], t["pprobs"], sc.fx, sc.fy, sc.px, sc.py,
                           t["view"], (200_000, 200_000), (16, 16), 1.0, 1000.0)
    torch.cuda.synchronize()
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    _, field, (fT, nc, pl, ranges, vis) = _run_gpu_forward(sc)
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
    assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL


def test_backward_prologue_on_a_second_stream(hrf):
    """Frame.backward queues the rasterizer backward's prologue (accumulator
    clear, block order) on a second stream beside the propagation adjoint
    (hrf_raster_backward_prepare); the backward then waits for it.  Its
    gradients equal those of a backward that runs its own prologue (up to
    the order of float atomics), over two frames in a row; a prepared
    workspace followed by a backward of another configuration (no plane
    lists) runs its own prologue and gives the same gradients."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import propagation, rasterizer, scenes
    from complex_valued_holographic_radiance_fields_amd.frame import Frame
    from complex_valued_holographic_radiance_fields_amd.scenes import FAR, NEAR, PITCH

    spec = scenes.small("prep", 8000, 128, 128, 3, 3, "object", seed=5)
    sc = scenes.generate(spec)
    t = scenes.to_torch(sc)
    fr = Frame(t, spec, sc.fx, sc.fy, sc.px, sc.py)
    g = torch.randn((len(spec.wavelengths), spec.size, spec.size), dtype=torch.complex64,
                    device="cuda")
    args = (t["cam_means"], t["z"], t["quats"], t["scales"], t["colours"], t["phase"], t["opac"],
            t["pprobs"], sc.fx, sc.fy, sc.px, sc.py, t["view"], (spec.width, spec.height))
    for frame in range(2):
        fr.forward()
        got = fr.backward(g)
        torch.cuda.synchronize()
        final_T, n_contrib, point_list, ranges, _ = fr.fwd_state
        gf = propagation.multiplane_adjoint(g, (spec.height, spec.width), spec.wavelengths,
                                            PITCH, [-d for d in spec.distances],
                                            (spec.size, spec.size), float(spec.size))
        ref = rasterizer.backward(gf, *args, (16, 16), final_T, n_contrib, point_list, ranges,
                                  NEAR, FAR, geometry=fr.geometry)
        torch.cuda.synchronize()
        errs = [rel_l2(a.cpu().numpy(), b.cpu().numpy()) for a, b in zip(got, ref)]
        print(f"frame {frame}: prepared vs own prologue, rel-L2 per gradient "
              f"{['%.1e' % e for e in errs]}", flush=True)
        assert max(errs) < 1e-6
    # prepared for the plane lists, then a backward without them
    rasterizer.backward_prepare(*args, point_list, NEAR, FAR, geometry=fr.geometry)
    other = rasterizer.backward(gf, *args, (16, 16), final_T, n_contrib, point_list, ranges,
                                NEAR, FAR, geometry=fr.geometry.workspace)
    torch.cuda.synchronize()
    errs = [rel_l2(a.cpu().numpy(), b.cpu().numpy()) for a, b in zip(other, ref)]
    print(f"mismatched preparation: rel-L2 per gradient {['%.1e' % e for e in errs]}", flush=True)
    assert max(errs) < 1e-6


def _tag_scene(case):
    """Scenes for the pair-tag path: needle-like Gaussians (one axis e^-2.5,
    the others e^-6) whose 3-sigma tile rectangles hold many tiles they never
    reach, soft plane weights (several planes per Gaussian, some below the
    cutoff), or opaque ones where most pixels terminate."""
    from complex_valued_holographic_radiance_fields_amd import scenes

    P, C = (1, 1) if case == "p1c1" else (3, 3)
    spec = scenes.SceneSpec("tags", 12, 20_000, 384, 320, P, [639e-9, 515e-9, 473e-9][:C],
                            [-1e-3, 0.0, 1e-3][:P], "uniform", log_scale_mean=-6.0,
                            log_scale_std=0.5)
    sc = scenes.generate(spec)
    rng = np.random.default_rng(5)
    m = sc.scales.shape[0]
    sc.scales[:, 0] = np.exp(rng.normal(-2.5, 0.5, size=m)).astype(np.float32)
    if case == "soft":
        w = rng.uniform(0, 1, size=sc.pprobs.shape).astype(np.float32)
        w[rng.uniform(size=w.shape) < 0.4] = 0.0
        w[rng.uniform(size=w.shape) < 0.05] = 5e-7
        sc.pprobs[:] = w
    if case == "dense":
        sc.scales[:, 1:] *= np.float32(np.exp(1.5))
        sc.opac[:] = 0.97
    return sc


@pytest.mark.parametrize("case", ["needles", "soft", "dense", "p1c1"])
def test_tagged_pair_lists(hrf, oracle_mod, monkeypatch, case):
    """Pair tags (wide keys whose first sort pass regenerates the pairs: the
    emission tests each (tile, gaussian) pair as the forward's visibility cull
    would, the last pass writes the result beside point_list, and the
    forward skips the untagged entries unseen).  Forced here at small sizes
    (HRF_SORT_VBITS widens the gaussian field past one word,
    HRF_SORT_REGENERATE takes the regenerating first pass).  Binning against
    the oracle bit for bit; field, final_T, n_contrib and the plane member
    lists as the untagged path's (the tags only skip what that path culls; the
    batches differ, so to rounding); field and the 8 gradients (backward on
    the tagged forward's plane lists) against the oracle."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import rasterizer

    sc = _tag_scene(case)
    g, cam = oracle_inputs(sc)
    ref = oracle_mod.rasterize_forward(g, cam)
    W, H = sc.spec.width, sc.spec.height
    t = scenes_torch(sc)
    args = (t["cam_means"], t["z"], t["quats"], t["scales"], t["colours"], t["phase"], t["opac"],
            t["pprobs"], sc.fx, sc.fy, sc.px, sc.py, t["view"])

    def run():
        out = rasterizer.forward(*args, (W, H), (16, 16), 1.0, 1000.0, keep_geometry=True)
        torch.cuda.synchronize()
        return out

    plain_field, plain_info, plain_geom = run()
    monkeypatch.setenv("HRF_SORT_VBITS", "24")
    monkeypatch.setenv("HRF_SORT_REGENERATE", "1")
    field, info, geom = run()
    monkeypatch.delenv("HRF_SORT_VBITS")
    monkeypatch.delenv("HRF_SORT_REGENERATE")
    fT, nc, pl, ranges, vis = info
    K = int(pl.numel())
    done = float((fT < 1e-4).float().mean())
    print(f"tags {case}: N={g.n} K={K} terminated={done:.3f}", flush=True)
    np.testing.assert_array_equal(ranges.cpu().numpy(), ref["ranges"])
    np.testing.assert_array_equal(pl.cpu().numpy(), ref["point_list"])
    np.testing.assert_array_equal(vis.cpu().numpy(), ref["visible"])
    # Against the untagged path: the tagged walk stages its candidates in
    # other batches (so a batch's choice of the reference-order or the fast
    # exponent may differ: rounding only), and may stop one window later.
    assert rel_l2(field.cpu().numpy(), plain_field.cpu().numpy()) < 1e-6
    assert rel_l2(fT.cpu().numpy(), plain_info[0].cpu().numpy()) < 1e-6
    assert np.mean(nc.cpu().numpy() != plain_info[1].cpu().numpy()) < 1e-3
    # plane member lists: per (tile, plane) the same entries in the same
    # order up to the shorter list's count (the buffer past a count is
    # scratch)
    P = g.P
    ntiles = ranges.shape[0]
    c0 = (P * K * 8 + 255) // 256 * 256
    lists = []
    for gm in (geom, plain_geom):
        buf = gm.plane_lists.cpu().numpy()
        ent = buf[:P * K * 8].view(np.int64).reshape(P, K)
        cnt = buf[c0:c0 + ntiles * P * 4].view(np.int32).reshape(ntiles, P)
        lists.append((ent, cnt))
    r_np = ranges.cpu().numpy()
    for tile in range(ntiles):
        for p in range(P):
            a = r_np[tile, 0]
            c = min(lists[0][1][tile, p], lists[1][1][tile, p])
            np.testing.assert_array_equal(lists[0][0][p, a:a + c], lists[1][0][p, a:a + c])
    assert rel_l2(field.cpu().numpy(), ref["field"]) < TOL
    assert rel_l2(fT.cpu().numpy(), ref["final_T"]) < TOL
    assert np.mean(nc.cpu().numpy() != ref["n_contrib"]) < 1e-3
    if case == "dense":
        assert done > 0.2
    else:
        assert done < 0.9

    rng = np.random.default_rng(6)
    gf = ((rng.normal(size=field.shape) + 1j * rng.normal(size=field.shape)) *
          np.sqrt(0.5)).astype(np.complex64)
    grads = rasterizer.backward(torch.from_numpy(gf).cuda(), *args, (W, H), (16, 16), fT, nc, pl,
                                ranges, 1.0, 1000.0, geometry=geom)
    torch.cuda.synchronize()
    state = dict(ref, final_T=fT.cpu().numpy(), n_contrib=nc.cpu().numpy())
    rb = oracle_mod.rasterize_backward(g, cam, state, gf)
    names = ["cam", "z", "quats", "scales", "colours", "phase", "opac", "plane"]
    for name, a in zip(names, grads):
        if name == "z":
            continue
        err = rel_l2(a.cpu().numpy(), rb[name])
        print(f"tags {case} grad_{name}: rel_l2={err:.3e}", flush=True)
        assert err < TOL, (name, err)
