"""The CPU baseline's restatement of the reference's CPU PyTorch path
(oracle/cpu_baseline.py; timing only, never the product): the explicit
adjoint of the pure-torch ASM against torch autograd of the forward, and the
tile-by-tile whole-frame runner (the backward one 64x64 tile at a time, so
large frames fit in host memory) against the whole-graph runner."""
import numpy as np
import pytest
import torch

from conftest import rel_l2


def test_asm_adjoint_matches_autograd():
    from oracle import cpu_baseline as cb

    gen = torch.Generator().manual_seed(3)
    H, W, S = 24, 20, 32
    x = torch.complex(torch.randn(H, W, generator=gen), torch.randn(H, W, generator=gen))
    g = torch.complex(torch.randn(S, S, generator=gen), torch.randn(S, S, generator=gen))
    for d in (-1e-3, 2e-4):
        xr = x.clone().requires_grad_(True)
        out = cb.asm_torch(xr, 532e-9, 3.74e-6, d, S, float(S) * 0.8)
        (out.real * g.real + out.imag * g.imag).sum().backward()
        adj = cb.asm_torch_adjoint(g, 532e-9, 3.74e-6, d, S, float(S) * 0.8, H, W)
        # autograd's gradient of Re<A x, g> w.r.t. x is A^H g
        assert rel_l2(adj.numpy(), xr.grad.numpy()) < 1e-5, d
        # and the adjoint identity Re<A x, g> = Re<x, A^H g>
        lhs = float((out.detach().conj() * g).sum().real)
        rhs = float((x.conj() * adj).sum().real)
        assert abs(lhs - rhs) <= 1e-4 * abs(lhs)


def test_tiled_frame_matches_whole_graph():
    from complex_valued_holographic_radiance_fields_amd import scenes
    from oracle import cpu_baseline as cb

    spec = scenes.small("cpu_tiled", 600, 96, 80, 2, 3, "object", seed=5)
    sc = scenes.generate(spec)
    torch.set_num_threads(4)
    whole = cb.run_frame(sc, backward=True)
    tiled = cb.run_frame_tiled(sc)
    assert whole["finished"] and tiled["finished"]
    assert tiled["tiles_done"] == tiled["tiles"] == 4
    assert rel_l2(tiled["hologram"].numpy(), whole["hologram"].numpy()) < 1e-5
    for a, b in zip(tiled["grads"], whole["grads"]):
        assert a is not None and b is not None
        assert rel_l2(a.numpy(), b.numpy()) < 1e-4
    assert np.isfinite(tiled["fwd_ms"]) and np.isfinite(tiled["bwd_ms"])
