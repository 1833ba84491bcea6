"""The BASELINE configurations at full size, checked through properties that
do not need the oracle's full render (which is too slow at these sizes):

* binning: `ranges` partition [0, K) in tile order with empty tiles (0, 0);
  every Gaussian appears exactly tiles_touched times (the oracle's
  preprocess, cheap on the CPU); every pair's tile lies in its Gaussian's
  tile rectangle; within a tile the pairs are ordered by (depth key, index) —
  together these fix point_list exactly;
* render: fields and gradients finite, final_T in (0, 1], n_contrib no
  larger than the tile's list;
* propagation at the configuration's grid: the adjoint identity
  <A x, y> = <x, A^H y> (cfg4's 3840 grid runs the fused LDS-FFT passes).

cfg4 (3M Gaussians at 1920x1080, ~8.7e8 pairs) also exercises the key/value
sort path (tile and gaussian bits do not fit one 32-bit word); the headline
geometry with larger Gaussians (2.4e7 pairs) runs the packed sort with several
key tiles per scatter block; a 160 x 125-tile grid with 150k Gaussians runs the
key/value sort with ranges formed from the sorted tiles; 8.3e7 pairs run the
packed sort over the larger (8192-key) tiles."""
import numpy as np
import pytest

from conftest import oracle_inputs, rel_l2

pytestmark = pytest.mark.gpu

CHUNK = 1 << 26


def _depth_key(z):
    import torch

    b = z.view(torch.int32).long() & 0xFFFFFFFF
    return torch.where((b & 0x80000000) != 0, b & 0x7FFFFFFF, b | 0x80000000)


def _check_binning(t, pl, ranges, tiles_ref, rect_ref, gx, ntiles):
    import torch

    dev = pl.device
    n = t["z"].numel()
    K = pl.numel()
    assert K == int(tiles_ref.astype(np.int64).sum())
    r = ranges.long()
    nonempty = r[:, 1] > r[:, 0]
    assert bool((r[~nonempty] == 0).all())
    starts, ends = r[nonempty, 0], r[nonempty, 1]
    assert int(starts[0]) == 0 and int(ends[-1]) == K
    assert torch.equal(starts[1:], ends[:-1])
    cnt = torch.bincount(pl.long(), minlength=n)
    assert torch.equal(cnt.cpu(), torch.from_numpy(tiles_ref.astype(np.int64)))
    tile_ids = torch.arange(ntiles, device=dev)[nonempty]
    seg_len = ends - starts
    key = _depth_key(t["z"])
    rect = torch.from_numpy(rect_ref.astype(np.int64)).to(dev)
    # Walk the pairs in chunks: tile of each position, rectangle membership,
    # (depth key, index) order inside each tile.
    seg_end = torch.cumsum(seg_len, 0)
    for c0 in range(0, K, CHUNK):
        c1 = min(K, c0 + CHUNK + 1)
        pos = torch.arange(c0, c1, device=dev)
        seg = torch.searchsorted(seg_end, pos, right=True)
        tile = tile_ids[seg]
        g = pl[c0:c1].long()
        tx, ty = tile % gx, tile // gx
        rg = rect[g]
        assert bool(((tx >= rg[:, 0]) & (tx < rg[:, 2]) & (ty >= rg[:, 1]) & (ty < rg[:, 3])).all())
        same = tile[1:] == tile[:-1]
        k0, k1 = key[g[:-1]], key[g[1:]]
        ordered = (k0 < k1) | ((k0 == k1) & (g[:-1] < g[1:]))
        assert bool((ordered | ~same).all())


@pytest.mark.parametrize("name", ["cfg1", "cfg2", "cfg4"])
def test_config_full_size(hrf, oracle_mod, name):
    import torch
    from complex_valued_holographic_radiance_fields_amd import scenes
    from complex_valued_holographic_radiance_fields_amd.frame import Frame

    spec = scenes.config(name)
    sc = scenes.generate(spec)
    g, cam = oracle_inputs(sc)
    pr = oracle_mod.project(g, cam)
    _, tiles_ref, rect_ref = oracle_mod.preprocess(pr["means2d"], pr["cov2d"], g.z, cam)
    print(f"{name}: N={g.n} K={int(tiles_ref.astype(np.int64).sum())}", flush=True)
    t = scenes.to_torch(sc)
    fr = Frame(t, spec, sc.fx, sc.fy, sc.px, sc.py)
    holo = fr.forward()
    grads = fr.backward(t["grad_holo"])
    torch.cuda.synchronize()
    fT, nc, pl, ranges, vis = fr.fwd_state
    W, H = spec.width, spec.height
    gx, gy = (W + 15) // 16, (H + 15) // 16
    _check_binning(t, pl, ranges, tiles_ref, rect_ref, gx, gx * gy)
    assert bool(torch.isfinite(torch.view_as_real(fr.fields)).all())
    assert bool(torch.isfinite(torch.view_as_real(holo)).all())
    assert bool(((fT > 0) & (fT <= 1)).all())
    # n_contrib never exceeds the pixel's tile list length
    r = ranges.long()
    lens = (r[:, 1] - r[:, 0]).reshape(gy, gx)
    tile_len = lens.repeat_interleave(16, 0).repeat_interleave(16, 1)[:H, :W]
    assert bool((nc.long() <= tile_len.unsqueeze(0)).all())
    for gg in grads:
        assert bool(torch.isfinite(gg).all())
    del fr, holo, grads
    torch.cuda.empty_cache()


@pytest.mark.parametrize("name", ["headline", "cfg2", "cfg4"])
def test_config_propagation_adjoint(hrf, name):
    import torch
    from complex_valued_holographic_radiance_fields_amd import propagation, scenes

    spec = scenes.config(name)
    P, C, H, W, S = spec.planes, len(spec.wavelengths), spec.height, spec.width, spec.size
    gen = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn((P, C, H, W), dtype=torch.complex64, device="cuda", generator=gen)
    y = torch.randn((C, S, S), dtype=torch.complex64, device="cuda", generator=gen)
    dist = [-d for d in spec.distances]
    print(f"{name}: grid {2 * S}", flush=True)
    Ax = propagation.multiplane(x, spec.wavelengths, scenes.PITCH, dist, (S, S), float(S))
    Ahy = propagation.multiplane_adjoint(y, (H, W), spec.wavelengths, scenes.PITCH, dist, (S, S),
                                         float(S))
    lhs = torch.vdot(Ax.reshape(-1).to(torch.complex128), y.reshape(-1).to(torch.complex128))
    rhs = torch.vdot(x.reshape(-1).to(torch.complex128), Ahy.reshape(-1).to(torch.complex128))
    assert float(abs(lhs - rhs) / abs(lhs)) < 1e-5


def test_cfg3_propagation_microbench(hrf, oracle_mod):
    """Config 3 at full size: (3, 2048, 2048) fields to 8 log-spaced
    distances on the 4096 grid (fused LDS-FFT passes), forward and adjoint.
    One (distance, channel) output is checked against the oracle (numpy
    double-precision FFT); the full operator through the adjoint identity."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import propagation, scenes

    field, wl, dist = scenes.cfg3_fields()
    C, S = field.shape[0], field.shape[1]
    print(f"cfg3: C={C} S={S} grid {2 * S} D={len(dist)}", flush=True)
    x = torch.from_numpy(field).cuda()
    out = propagation.multidistance(x, wl, scenes.PITCH, dist, (S, S), float(S))
    torch.cuda.synchronize()
    assert tuple(out.shape) == (len(dist), C, S, S)
    assert bool(torch.isfinite(torch.view_as_real(out)).all())
    d, c = 5, 1
    ref = oracle_mod.asm_forward(field[c], wl[c], scenes.PITCH, dist[d], S, float(S))
    assert rel_l2(out[d, c].cpu().numpy(), ref) < 1e-4
    gen = torch.Generator(device="cuda").manual_seed(5)
    y = torch.randn(tuple(out.shape), dtype=torch.complex64, device="cuda", generator=gen)
    Ahy = propagation.multidistance_adjoint(y, (S, S), wl, scenes.PITCH, dist, (S, S), float(S))
    lhs = torch.vdot(out.reshape(-1).to(torch.complex128), y.reshape(-1).to(torch.complex128))
    rhs = torch.vdot(x.reshape(-1).to(torch.complex128), Ahy.reshape(-1).to(torch.complex128))
    assert float(abs(lhs - rhs) / abs(lhs)) < 1e-5
    del out, y, Ahy
    torch.cuda.empty_cache()


def test_packed_sort_partitioned(hrf, oracle_mod):
    """The headline geometry with larger Gaussians (log-scale mean -3.5): K
    above 2^24 pairs with tile and gaussian still in one 32-bit word, so the
    packed sort's passes run with several 2048-key tiles per block and the
    last pass writes point_list; binning checked exactly as above."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import scenes
    from complex_valued_holographic_radiance_fields_amd.frame import Frame

    base = scenes.config("headline")
    spec = scenes.SceneSpec("packed_big", 9, base.n, base.width, base.height, base.planes,
                            base.wavelengths, base.distances, "object", log_scale_mean=-3.5)
    sc = scenes.generate(spec)
    g, cam = oracle_inputs(sc)
    pr = oracle_mod.project(g, cam)
    _, tiles_ref, rect_ref = oracle_mod.preprocess(pr["means2d"], pr["cov2d"], g.z, cam)
    K = int(tiles_ref.astype(np.int64).sum())
    print(f"packed_big: N={g.n} K={K}", flush=True)
    assert K > (1 << 24)
    t = scenes.to_torch(sc)
    fr = Frame(t, spec, sc.fx, sc.fy, sc.px, sc.py)
    fr.forward()
    torch.cuda.synchronize()
    fT, nc, pl, ranges, vis = fr.fwd_state
    W, H = spec.width, spec.height
    gx, gy = (W + 15) // 16, (H + 15) // 16
    _check_binning(t, pl, ranges, tiles_ref, rect_ref, gx, gx * gy)
    assert bool(((fT > 0) & (fT <= 1)).all())
    del fr
    torch.cuda.empty_cache()


def test_wide_sort_path_large_grid(hrf, oracle_mod):
    """A tile grid beyond the difference array's bound (160 x 125 tiles) with
    150k Gaussians: tile (15) and gaussian (18) bits exceed one word, so the
    pairs go through the key/value sort and the ranges are formed from the
    sorted tiles (the path the direct binning does not take); binning checked
    exactly as above."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import scenes
    from complex_valued_holographic_radiance_fields_amd.frame import Frame

    spec = scenes.SceneSpec("wide_grid", 11, 150_000, 2560, 2000, 1, [515e-9], [-2e-3],
                            "uniform")
    sc = scenes.generate(spec)
    g, cam = oracle_inputs(sc)
    pr = oracle_mod.project(g, cam)
    _, tiles_ref, rect_ref = oracle_mod.preprocess(pr["means2d"], pr["cov2d"], g.z, cam)
    print(f"wide_grid: N={g.n} K={int(tiles_ref.astype(np.int64).sum())}", flush=True)
    t = scenes.to_torch(sc)
    fr = Frame(t, spec, sc.fx, sc.fy, sc.px, sc.py)
    fr.forward()
    torch.cuda.synchronize()
    fT, nc, pl, ranges, vis = fr.fwd_state
    gx, gy = (spec.width + 15) // 16, (spec.height + 15) // 16
    assert (gx + 1) * (gy + 1) > 16000
    _check_binning(t, pl, ranges, tiles_ref, rect_ref, gx, gx * gy)
    assert bool(((fT > 0) & (fT <= 1)).all())
    del fr
    torch.cuda.empty_cache()


def test_packed_sort_first_pass_from_emission(hrf, oracle_mod):
    """100k large Gaussians at 800x800 (3.3e7 pairs, ~8e4 per emission block):
    the emission takes the packed sort's first-pass histogram over its own
    blocks, which become that pass's partitions; binning checked exactly."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import scenes
    from complex_valued_holographic_radiance_fields_amd.frame import Frame

    spec = scenes.SceneSpec("first_pass", 12, 100_000, 800, 800, 1, [515e-9], [-2e-3], "object",
                            log_scale_mean=-2.0)
    sc = scenes.generate(spec)
    g, cam = oracle_inputs(sc)
    pr = oracle_mod.project(g, cam)
    _, tiles_ref, rect_ref = oracle_mod.preprocess(pr["means2d"], pr["cov2d"], g.z, cam)
    K = int(tiles_ref.astype(np.int64).sum())
    print(f"first_pass: N={g.n} K={K}", flush=True)
    assert K // ((g.n + 255) // 256) >= 16 * 2048
    t = scenes.to_torch(sc)
    fr = Frame(t, spec, sc.fx, sc.fy, sc.px, sc.py)
    fr.forward()
    torch.cuda.synchronize()
    fT, nc, pl, ranges, vis = fr.fwd_state
    gx, gy = (spec.width + 15) // 16, (spec.height + 15) // 16
    _check_binning(t, pl, ranges, tiles_ref, rect_ref, gx, gx * gy)
    del fr
    torch.cuda.empty_cache()


def test_packed_sort_large_tiles(hrf, oracle_mod):
    """250k large Gaussians at 800x800 (8.3e7 pairs, above the 2^26 keys from
    which the sort passes run 1024-thread blocks over 8192-key tiles): the
    first pass over the emission's partitions and the second with its own
    histogram both run the larger tiles; binning checked exactly."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import scenes
    from complex_valued_holographic_radiance_fields_amd.frame import Frame

    spec = scenes.SceneSpec("large_tiles", 13, 250_000, 800, 800, 1, [515e-9], [-2e-3],
                            "object", log_scale_mean=-2.0)
    sc = scenes.generate(spec)
    g, cam = oracle_inputs(sc)
    pr = oracle_mod.project(g, cam)
    _, tiles_ref, rect_ref = oracle_mod.preprocess(pr["means2d"], pr["cov2d"], g.z, cam)
    K = int(tiles_ref.astype(np.int64).sum())
    print(f"large_tiles: N={g.n} K={K}", flush=True)
    assert K >= (1 << 26)
    t = scenes.to_torch(sc)
    fr = Frame(t, spec, sc.fx, sc.fy, sc.px, sc.py)
    fr.forward()
    torch.cuda.synchronize()
    fT, nc, pl, ranges, vis = fr.fwd_state
    gx, gy = (spec.width + 15) // 16, (spec.height + 15) // 16
    _check_binning(t, pl, ranges, tiles_ref, rect_ref, gx, gx * gy)
    assert bool(((fT > 0) & (fT <= 1)).all())
    del fr
    torch.cuda.empty_cache()
