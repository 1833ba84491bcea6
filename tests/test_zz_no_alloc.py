"""hrf_grad_norm_static, the allocation-free variant of hrf_grad_norm (its
partial sums live in the library's static device array): through the C ABI,
its norm and clip coefficient equal hrf_grad_norm's (same kernels, same
summation order: bit for bit) on two calls in a row, the second with a
smaller input, so nothing of the first call's partial sums can leak into
the second; and both agree with torch's clip_grad_norm_ arithmetic."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _norm_both(L, lib, grads, max_norm):
    import torch

    n = len(grads)
    ptrs = (ctypes.c_void_p * n)(*[g.data_ptr() for g in grads])
    numels = (ctypes.c_int64 * n)(*[g.numel() for g in grads])
    dev = grads[0].device
    stream = L.stream_ptr(dev)
    out = torch.full((4,), -1.0, device=dev)
    wsb = lib.hrf_grad_norm_workspace_size(numels, n)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    L.check(lib.hrf_grad_norm(ptrs, numels, n, max_norm, out[0:].data_ptr(),
                              out[1:].data_ptr(), ws.data_ptr(), wsb, stream))
    L.check(lib.hrf_grad_norm_static(ptrs, numels, n, max_norm, out[2:].data_ptr(),
                                     out[3:].data_ptr(), stream))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_grad_norm_static_matches_workspace_entry(hrf):
    import torch
    from complex_valued_holographic_radiance_fields_amd import _lib as L

    lib = L.load()
    gen = torch.Generator(device="cuda").manual_seed(11)
    # first call: seven tensors of the headline's parameter shapes (N = 1M):
    # 20M elements, 9770 partial sums
    shapes = [(1_000_000, k) for k in (3, 3, 3, 3, 1, 3, 4)]
    big = [torch.randn(s, generator=gen, device="cuda") * 0.01 for s in shapes]
    o1 = _norm_both(L, lib, big, 1.0)
    print(f"call 1: norm {o1[0]:.6f} / {o1[2]:.6f}, coef {o1[1]:.6g} / {o1[3]:.6g}", flush=True)
    assert o1[0] == o1[2] and o1[1] == o1[3]
    ref = torch.linalg.vector_norm(torch.stack([torch.linalg.vector_norm(g.double())
                                                for g in big]))
    assert abs(float(o1[0]) - float(ref)) <= 1e-5 * float(ref)
    assert abs(float(o1[1]) - min(1.0, 1.0 / (float(ref) + 1e-6))) <= 1e-5
    # second call, smaller: three small tensors (a few partial sums); the
    # first call's partials beyond them must not count
    small = [torch.randn(s, generator=gen, device="cuda") for s in ((5000, 3), (777,), (64, 9))]
    o2 = _norm_both(L, lib, small, 2.5)
    print(f"call 2: norm {o2[0]:.6f} / {o2[2]:.6f}, coef {o2[1]:.6g} / {o2[3]:.6g}", flush=True)
    assert o2[0] == o2[2] and o2[1] == o2[3]
    ref2 = float(np.sqrt(sum(float((g.double() ** 2).sum()) for g in small)))
    assert abs(float(o2[0]) - ref2) <= 1e-5 * ref2
    assert abs(float(o2[1]) - min(1.0, 2.5 / (ref2 + 1e-6))) <= 1e-6
    # a third call with the first input again gives the first result
    o3 = _norm_both(L, lib, big, 1.0)
    assert o3[2] == o1[0] and o3[3] == o1[1]


def test_grad_norm_static_allocates_nothing_and_replays_in_a_graph(hrf):
    """The reasons the entry point exists: free device memory (hipMemGetInfo,
    through torch.cuda.mem_get_info) is the same before and after calls once
    the device's array address is known, and the call captured into a HIP
    graph (after one call on the device) replays correctly: each replay, with
    new gradient values written eagerly between replays, equals the
    workspace entry point run eagerly on the same values, bit for bit."""
    import torch
    from complex_valued_holographic_radiance_fields_amd import _lib as L

    lib = L.load()
    gen = torch.Generator(device="cuda").manual_seed(23)
    grads = [torch.empty(s, device="cuda") for s in ((300_000, 3), (300_000,), (4097,))]
    for g in grads:
        g.copy_(torch.randn(g.shape, generator=gen, device="cuda"))
    n = len(grads)
    ptrs = (ctypes.c_void_p * n)(*[g.data_ptr() for g in grads])
    numels = (ctypes.c_int64 * n)(*[g.numel() for g in grads])
    out = torch.zeros(2, device="cuda")

    def static_call():
        L.check(lib.hrf_grad_norm_static(ptrs, numels, n, 1.5, out[0:].data_ptr(),
                                         out[1:].data_ptr(), L.stream_ptr(out.device)))

    static_call()  # the device's array address is looked up here
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(3):
        static_call()
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    print(f"free device memory before/after three calls: {free0} / {free1}", flush=True)
    assert free1 == free0

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        static_call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        static_call()
    torch.cuda.synchronize()
    for rep in range(4):
        for g in grads:
            g.copy_(torch.randn(g.shape, generator=gen, device="cuda") * (rep + 1))
        torch.cuda.synchronize()
        out.fill_(-1.0)
        graph.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy().copy()
        ref = _norm_both(L, lib, grads, 1.5)
        print(f"replay {rep}: norm {got[0]:.6f} (eager {ref[0]:.6f}), coef {got[1]:.6g} "
              f"(eager {ref[1]:.6g})", flush=True)
        assert got[0] == ref[0] and got[1] == ref[1]
        assert got[0] == ref[2] and got[1] == ref[3]
