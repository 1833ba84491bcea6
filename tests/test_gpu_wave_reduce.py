"""Lane layout of the wave64 reductions used by the backward render kernel."""
import ctypes
import os

import numpy as np
import pytest

from conftest import REPO

pytestmark = pytest.mark.gpu

LIB = os.path.join(REPO, "tests", "hip", "libwave_test.so")


@pytest.fixture(scope="module")
def wlib(hrf):
    lib = ctypes.CDLL(LIB)
    for f in (lib.wave_test_transpose, lib.wave_test_sum, lib.wave_test_row_sum16):
        f.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        f.restype = ctypes.c_int
    return lib


def test_transpose_reduce64(wlib):
    import torch

    rng = np.random.default_rng(0)
    x = rng.integers(-1000, 1000, size=(64, 64)).astype(np.float32)  # exact sums
    xin = torch.from_numpy(x).cuda()
    out = torch.zeros(64, dtype=torch.float32, device="cuda")
    assert wlib.wave_test_transpose(xin.data_ptr(), out.data_ptr()) == 0
    np.testing.assert_array_equal(out.cpu().numpy(), x.sum(axis=0))


def test_row_sum16(wlib):
    """Each lane L ends with the 16-lane row sums of values 6 b3 + 3 b2 + i
    (b3, b2 = bits 3 and 2 of L), i = 0..2."""
    import torch

    rng = np.random.default_rng(1)
    x = rng.integers(-1000, 1000, size=(64, 12)).astype(np.float32)  # exact sums
    xin = torch.from_numpy(x).cuda()
    out = torch.zeros(64 * 3, dtype=torch.float32, device="cuda")
    assert wlib.wave_test_row_sum16(xin.data_ptr(), out.data_ptr()) == 0
    got = out.cpu().numpy().reshape(64, 3)
    rows = x.reshape(4, 16, 12).sum(axis=1)  # (row, value)
    lane = np.arange(64)
    idx = 6 * ((lane >> 3) & 1)[:, None] + 3 * ((lane >> 2) & 1)[:, None] + np.arange(3)[None, :]
    np.testing.assert_array_equal(got, rows[lane[:, None] // 16, idx])


def test_wave_sum_lane63(wlib):
    import torch

    x = np.arange(64, dtype=np.float32) * 3 - 50
    xin = torch.from_numpy(x).cuda()
    out = torch.zeros(64, dtype=torch.float32, device="cuda")
    assert wlib.wave_test_sum(xin.data_ptr(), out.data_ptr()) == 0
    assert out[63].item() == x.sum()


def test_sincos_big_accuracy(wlib):
    """sin/cos of the transfer-function phase (float arguments up to 1e5 rad,
    as d*kz reaches) against float64 sin/cos of the same float values."""
    import torch

    f = wlib.trig_test_sincos
    f.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int]
    f.restype = ctypes.c_int
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.uniform(-1e5, 1e5, 200_000), rng.uniform(-10, 10, 50_000),
                        np.array([0.0, np.pi, -np.pi, 2 * np.pi, 1e5])]).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    s = torch.empty_like(xt)
    c = torch.empty_like(xt)
    assert f(xt.data_ptr(), s.data_ptr(), c.data_ptr(), x.size) == 0
    xd = x.astype(np.float64)
    err = max(np.abs(s.cpu().numpy() - np.sin(xd)).max(), np.abs(c.cpu().numpy() - np.cos(xd)).max())
    print(f"sincos_big max abs error {err:.2e}", flush=True)
    assert err < 2e-6
