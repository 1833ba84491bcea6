"""GPU parity of the HIP band-limited ASM against the oracle (C ABI path)."""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu

PITCH = 3.74e-6
TOL = 1e-4


def _field(rng, shape):
    amp = rng.uniform(0, 1, size=shape)
    ph = rng.uniform(0, 2 * np.pi, size=shape)
    return (amp * np.exp(1j * ph)).astype(np.complex64)


@pytest.mark.parametrize("M,d,ap", [(64, 1e-3, 32.0), (128, -2.5e-3, -1.0), (96, 4e-3, 48.0)])
@pytest.mark.parametrize("adjoint", [False, True])
def test_spectral_kernel_dropin(hrf, oracle_mod, M, d, ap, adjoint):
    """cuda_modules.bandlimited_propagation_{forward,backward} on FX/FY grids."""
    import torch
    from complex_valued_holographic_radiance_fields_amd.cuda_prop import cuda_module

    rng = np.random.default_rng(M)
    spec = _field(rng, (M, M)) * 100
    FX, FY = oracle_mod.freq_grids(M, PITCH)
    ore, oim = oracle_mod.asm_spectral(spec.real, spec.imag, FX, FY, 515e-9, d, ap, PITCH,
                                       adjoint=adjoint)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()  # noqa: E731
    if adjoint:
        gre, gim = cuda_module.bandlimited_propagation_backward(
            T(spec.real), T(spec.imag), T(spec.real), T(spec.imag), T(FX), T(FY), 515e-9, d, ap,
            PITCH)
    else:
        gre, gim = cuda_module.bandlimited_propagation_forward(
            T(spec.real), T(spec.imag), T(FX), T(FY), 515e-9, d, ap, PITCH)
    got = gre.cpu().numpy() + 1j * gim.cpu().numpy()
    assert rel_l2(got, ore + 1j * oim) < 1e-6


@pytest.mark.parametrize("H,W,S", [(48, 48, 48), (40, 56, 64), (256, 256, 256)])
@pytest.mark.parametrize("d", [2e-3, -1e-3, 0.0])
def test_single_propagation(hrf, oracle_mod, H, W, S, d):
    import torch
    from complex_valued_holographic_radiance_fields_amd.cuda_prop import BandlimitedPropagation

    rng = np.random.default_rng(H + W)
    f = _field(rng, (H, W))
    ref = oracle_mod.asm_forward(f, 515e-9, PITCH, d, S, float(S))
    ft = torch.from_numpy(f).cuda().requires_grad_(True)
    out = BandlimitedPropagation(ft, 515e-9, PITCH, d, [S, S], True, float(S))
    assert out.shape == (S, S)
    assert rel_l2(out.detach().cpu().numpy(), ref) < TOL
    g = _field(rng, (S, S))
    gt = torch.from_numpy(g).cuda()
    (out.real * gt.real + out.imag * gt.imag).sum().backward()
    ref_adj = oracle_mod.asm_adjoint(g, H, W, 515e-9, PITCH, d, S, float(S))
    assert rel_l2(ft.grad.cpu().numpy(), ref_adj) < TOL


def test_multiplane(hrf, oracle_mod):
    import torch
    from complex_valued_holographic_radiance_fields_amd import propagation

    rng = np.random.default_rng(3)
    P, C, H, W, S = 3, 3, 80, 64, 80
    wl = [639e-9, 515e-9, 473e-9]
    dist = [1e-3, 0.0, -1e-3]
    f = _field(rng, (P, C, H, W))
    ref = oracle_mod.multiplane_forward(f, wl, dist, PITCH, S, float(S))
    got = propagation.multiplane(torch.from_numpy(f).cuda(), wl, PITCH, dist, (S, S), float(S))
    assert rel_l2(got.cpu().numpy(), ref) < TOL
    g = _field(rng, (C, S, S))
    ref_adj = oracle_mod.multiplane_adjoint(g, H, W, wl, dist, PITCH, S, float(S))
    got_adj = propagation.multiplane_adjoint(torch.from_numpy(g).cuda(), (H, W), wl, PITCH, dist,
                                             (S, S), float(S))
    assert rel_l2(got_adj.cpu().numpy(), ref_adj) < TOL


def test_adjoint_identity(hrf):
    """<A x, y> == <x, A^H y> for the fused multi-plane operator."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import propagation

    rng = np.random.default_rng(9)
    P, C, H, W, S = 2, 3, 64, 64, 64
    wl = [639e-9, 515e-9, 473e-9]
    dist = [2e-3, -3e-3]
    x = torch.from_numpy(_field(rng, (P, C, H, W))).cuda()
    y = torch.from_numpy(_field(rng, (C, S, S))).cuda()
    Ax = propagation.multiplane(x, wl, PITCH, dist, (S, S), float(S))
    Ahy = propagation.multiplane_adjoint(y, (H, W), wl, PITCH, dist, (S, S), float(S))
    lhs = torch.vdot(Ax.reshape(-1).to(torch.complex128), y.reshape(-1).to(torch.complex128))
    rhs = torch.vdot(x.reshape(-1).to(torch.complex128), Ahy.reshape(-1).to(torch.complex128))
    assert abs(lhs - rhs) / abs(lhs) < 1e-5


def test_identity_at_zero_distance(hrf):
    """d = 0 with the aperture off is the identity (pad -> FFT -> iFFT -> crop)."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import propagation

    rng = np.random.default_rng(1)
    f = torch.from_numpy(_field(rng, (64, 64))).cuda()
    out = propagation.propagate(f, 515e-9, PITCH, 0.0, (64, 64), -1.0)
    assert rel_l2(out.cpu().numpy(), f.cpu().numpy()) < 1e-6


def test_odd_size_rejected(hrf):
    import torch
    from complex_valued_holographic_radiance_fields_amd import propagation

    f = torch.zeros((33, 32), dtype=torch.complex64, device="cuda")
    with pytest.raises(RuntimeError):
        propagation.propagate(f, 515e-9, PITCH, 1e-3, (64, 64), -1.0)


# Grids with a hand-written LDS-FFT plan (M = 2S in 128, 160, 192, 512, 1024,
# 1600, 2016, 2048, 3840, 4096) run the fused row/column kernels; other sizes
# (M = 96 above) run the hipFFT path.  The headline grid (800 -> 1600) and
# every large plan are checked against the oracle, forward and adjoint.
# Fields wider and/or taller than half the padded grid (up to 2S is allowed)
# take the transforms whose first stage is not pruned.
@pytest.mark.parametrize("P,C,H,W,S", [(3, 3, 800, 800, 800), (1, 2, 100, 60, 512),
                                       (2, 1, 64, 64, 1008), (1, 1, 128, 96, 1024),
                                       (2, 1, 120, 200, 1920), (1, 2, 96, 128, 2048),
                                       (1, 1, 40, 2300, 2048), (1, 1, 2000, 24, 1920),
                                       (1, 2, 96, 100, 64), (2, 1, 48, 120, 64),
                                       (1, 1, 110, 40, 80)],
                         ids=["headline1600", "m1024", "m2016", "m2048", "m3840", "m4096",
                              "wide_m4096", "tall_m3840", "wide_tall_m128", "wide_m128",
                              "tall_m160"])
def test_multiplane_fused_grids(hrf, oracle_mod, P, C, H, W, S):
    import torch
    from complex_valued_holographic_radiance_fields_amd import propagation

    rng = np.random.default_rng(S)
    wl = [639e-9, 515e-9, 473e-9][:C]
    dist = [-2e-3, -4e-3, -6e-3][:P]
    f = _field(rng, (P, C, H, W))
    print(f"fused grid M={2 * S} P={P} C={C}", flush=True)
    ref = oracle_mod.multiplane_forward(f, wl, dist, PITCH, S, float(S))
    got = propagation.multiplane(torch.from_numpy(f).cuda(), wl, PITCH, dist, (S, S), float(S))
    assert rel_l2(got.cpu().numpy(), ref) < TOL
    g = _field(rng, (C, S, S))
    ref_adj = oracle_mod.multiplane_adjoint(g, H, W, wl, dist, PITCH, S, float(S))
    got_adj = propagation.multiplane_adjoint(torch.from_numpy(g).cuda(), (H, W), wl, PITCH, dist,
                                             (S, S), float(S))
    assert rel_l2(got_adj.cpu().numpy(), ref_adj) < TOL


def test_fused_matches_hipfft_path(hrf):
    """At d = 0 with the aperture off, both transform paths reduce to
    pad -> FFT -> iFFT -> crop: the hipFFT path (M = 96) and the fused path
    (M = 128) must each give the input back."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import propagation

    rng = np.random.default_rng(4)
    f = torch.from_numpy(_field(rng, (48, 48))).cuda()
    a = propagation.propagate(f, 515e-9, PITCH, 0.0, (48, 48), -1.0)   # M = 96, hipFFT
    b = propagation.propagate(f, 515e-9, PITCH, 0.0, (64, 64), -1.0)   # M = 128, fused
    assert rel_l2(a.cpu().numpy(), f.cpu().numpy()) < 1e-6
    assert rel_l2(b[8:56, 8:56].cpu().numpy(), f.cpu().numpy()) < 1e-6


def test_fused_grid_with_active_band_limit(hrf, oracle_mod):
    """At 10-12 mm on a 128 grid (L = 0.48 mm) the band limit removes part of
    the spectrum (2d/L > 2 pitch / lambda), so the fused kernels take the
    per-element band test instead of the all-pass shortcut."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import propagation

    rng = np.random.default_rng(12)
    P, C, H, W, S = 2, 2, 48, 40, 64
    wl = [639e-9, 473e-9]
    dist = [10e-3, -12e-3]
    f = _field(rng, (P, C, H, W))
    ref = oracle_mod.multiplane_forward(f, wl, dist, PITCH, S, float(S))
    got = propagation.multiplane(torch.from_numpy(f).cuda(), wl, PITCH, dist, (S, S), float(S))
    assert rel_l2(got.cpu().numpy(), ref) < TOL
    g = _field(rng, (C, S, S))
    ref_adj = oracle_mod.multiplane_adjoint(g, H, W, wl, dist, PITCH, S, float(S))
    got_adj = propagation.multiplane_adjoint(torch.from_numpy(g).cuda(), (H, W), wl, PITCH, dist,
                                             (S, S), float(S))
    assert rel_l2(got_adj.cpu().numpy(), ref_adj) < TOL


def test_multidistance_matches_oracle(hrf, oracle_mod):
    """fields (C,H,W) to D distances with shared forward transforms: each
    out[d,c] is the oracle's single propagation; the adjoint is the sum of
    the single adjoints."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import propagation

    rng = np.random.default_rng(21)
    C, H, W, S = 2, 48, 40, 64
    wl = [639e-9, 473e-9]
    dist = [1e-4, 1.5e-3, -4e-3]
    f = _field(rng, (C, H, W))
    got = propagation.multidistance(torch.from_numpy(f).cuda(), wl, PITCH, dist, (S, S),
                                    float(S)).cpu().numpy()
    assert got.shape == (3, C, S, S)
    for d, dv in enumerate(dist):
        for c in range(C):
            ref = oracle_mod.asm_forward(f[c], wl[c], PITCH, dv, S, float(S))
            assert rel_l2(got[d, c], ref) < TOL, (d, c)
    g = _field(rng, (3, C, S, S))
    got_adj = propagation.multidistance_adjoint(torch.from_numpy(g).cuda(), (H, W), wl, PITCH,
                                                dist, (S, S), float(S)).cpu().numpy()
    for c in range(C):
        ref = sum(oracle_mod.asm_adjoint(g[d, c], H, W, wl[c], PITCH, dv, S, float(S))
                  for d, dv in enumerate(dist))
        assert rel_l2(got_adj[c], ref) < TOL, c


@pytest.mark.parametrize("S,D", [(48, 2), (64, 3), (96, 5)],
                         ids=["hipfft_m96", "fused_m128", "fused_m192"])
def test_multidistance_autograd_and_single_calls(hrf, S, D):
    """MultiDistancePropagation's backward is multidistance_adjoint, and every
    output equals the single-call propagation of the same field.  On the
    fused grids the distances go through the column passes two at a time
    (an odd count leaves a group of one)."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import propagation

    rng = np.random.default_rng(22)
    C, H, W = 3, 32, 32
    wl = [639e-9, 515e-9, 473e-9]
    dist = [2e-3, 5e-4, -1e-3, 3e-3, -2.5e-4][:D]
    f = torch.from_numpy(_field(rng, (C, H, W))).cuda().requires_grad_(True)
    out = propagation.MultiDistancePropagation.apply(f, wl, PITCH, dist, (S, S), float(S))
    for d, dv in enumerate(dist):
        for c in range(C):
            single = propagation.propagate(f.detach()[c], wl[c], PITCH, dv, (S, S), float(S))
            assert rel_l2(out.detach()[d, c].cpu().numpy(), single.cpu().numpy()) < 1e-6
    g = torch.from_numpy(_field(rng, (D, C, S, S))).cuda()
    (out.real * g.real + out.imag * g.imag).sum().backward()
    adj = propagation.multidistance_adjoint(g, (H, W), wl, PITCH, dist, (S, S), float(S))
    assert rel_l2(f.grad.cpu().numpy(), adj.cpu().numpy()) < 1e-6
