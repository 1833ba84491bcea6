"""Calibration kernels of known VALU work (tests/hip/wave_reduce_test.hip):
8192 waves, each issuing exactly 8 * iters v_fma_f32 (k_calib_fma) or
8 * iters v_exp_f32 + 8 * iters v_mul_f32 (k_calib_exp).  Run under
rocprofv3 --pmc, their SQ_INSTS_VALU / SQ_INSTS_VALU_TRANS_F32 /
SQ_ACTIVE_INST_VALU readings against these known counts calibrate the
counters the render kernels' VALU figures use; the printed issue rates
(wave-instructions per second, timed with hipEvents) give the measured
VALU and transcendental throughput of the card."""
import ctypes
import os

import pytest

from conftest import REPO

pytestmark = pytest.mark.gpu

LIB = os.path.join(REPO, "tests", "hip", "libwave_test.so")
BLOCKS = 2048  # x 4 waves = 8192 waves: 8 per SIMD on 256 CUs
ITERS = 4096


def _time_kernel(lib, kind, iters):
    import torch

    f = getattr(lib, f"calib_valu_{kind}")
    f.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_void_p]
    f.restype = ctypes.c_int
    out = torch.empty(BLOCKS * 256, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    assert f(out.data_ptr(), BLOCKS, 16, 0.5, stream) == 0  # warm-up
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ms = []
    for _ in range(3):
        e0.record()
        assert f(out.data_ptr(), BLOCKS, iters, 0.5, stream) == 0
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
    assert bool(torch.isfinite(out).all())
    return min(ms)


def test_transcendental_issue_cost_in_a_mix(hrf):
    """k_calib_mix issues 9 VALU instructions per iteration, one of them a
    v_exp_f32 independent of the 8 others; k_calib_fma issues 8 v_fma_f32.
    With every instruction taking one issue slot of its SIMD and the
    transcendental two, the mix takes 10/8 of the FMA kernel's time; if the
    transcendental overlaps the independent instructions, 9/8 (one slot).
    The printed cost per transcendental (in issue slots) is a measurement,
    not a property under test (timings under rocprofv3 counter collection
    are not meaningful), so only the outputs are checked."""
    lib = ctypes.CDLL(LIB)
    t_fma = _time_kernel(lib, "fma", ITERS)
    t_mix = _time_kernel(lib, "mix", ITERS)
    slot = t_fma / 8.0  # one issue slot per iteration per wave, in ms
    trans_slots = t_mix / slot - 8.0  # the mix's 9 instructions: 8 one-slot + 1 exp
    print(f"calib mix: fma {t_fma:.4f} ms (8 slots/iter), mix {t_mix:.4f} ms "
          f"-> a transcendental among independent VALU costs {trans_slots:.2f} issue slots",
          flush=True)
    t_fmac = _time_kernel(lib, "fmac", ITERS)
    print(f"calib fmac: VOP2 v_fmac_f32 {t_fmac:.4f} ms against VOP3 v_fma_f32 {t_fma:.4f} ms "
          f"for the same count", flush=True)


def test_forward_member_loop_rate(hrf):
    """k_calib_fwdloop runs the forward render's fast member loop (the same
    hrf::fwd_member, 8 members per all-done vote) over 256 staged members,
    64 times per wave, with no lane ever terminating: under rocprofv3 --pmc
    its SQ_INSTS_VALU over this time is the VALU issue rate the forward's
    instruction mix reaches by itself, the peak its VALU model uses."""
    lib = ctypes.CDLL(LIB)
    iters = 64
    ms = _time_kernel(lib, "fwdloop", iters)
    members = BLOCKS * 256 * iters * 256  # (pixel, member) evaluations
    print(f"calib fwdloop: {members / (ms * 1e-3) / 1e12:.3f} T pixel-member evaluations/s "
          f"({ms:.4f} ms for {BLOCKS * 4} waves x {iters * 256} members)", flush=True)


@pytest.mark.parametrize("kind", ["fma", "exp"])
def test_calibration_kernel_rates(hrf, kind):
    import torch

    lib = ctypes.CDLL(LIB)
    f = getattr(lib, f"calib_valu_{kind}")
    f.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_void_p]
    f.restype = ctypes.c_int
    out = torch.empty(BLOCKS * 256, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    assert f(out.data_ptr(), BLOCKS, 16, 0.5, stream) == 0  # warm-up
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    assert f(out.data_ptr(), BLOCKS, ITERS, 0.5, stream) == 0
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    waves = BLOCKS * 4
    per_wave = 8 * ITERS * (1 if kind == "fma" else 2)
    rate = waves * per_wave / (ms * 1e-3)
    print(f"calib {kind}: {waves} waves x {per_wave} VALU instructions in {ms:.4f} ms = "
          f"{rate / 1e9:.1f} G wave-instructions/s", flush=True)
    assert bool(torch.isfinite(out).all())
    assert rate > 1e11
