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
