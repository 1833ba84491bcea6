"""The oracle's own tests, rerun against its AddressSanitizer +
UndefinedBehaviorSanitizer build (oracle/Makefile `sanitized`: gcc, host
code only).  An out-of-bounds access, use after free, signed overflow,
misaligned load or out-of-range float-to-int conversion inside
hrf_oracle.c aborts the child run, which fails this test.

The child is a separate interpreter: the ASan runtime must be loaded before
anything else (LD_PRELOAD), and the sanitized library is selected with
HRF_ORACLE_LIB."""
import os
import subprocess
import sys

import pytest

from conftest import REPO

ORACLE = os.path.join(REPO, "oracle")


def _runtime(name):
    out = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
    path = out.stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


@pytest.mark.timeout(900)
def test_oracle_suite_under_asan_ubsan():
    asan = _runtime("libasan.so")
    if asan is None:
        pytest.skip("gcc's AddressSanitizer runtime is not installed")
    subprocess.run(["make", "-s", "-C", ORACLE, "sanitized"], check=True)
    env = dict(os.environ)
    env.update({
        "HRF_ORACLE_LIB": os.path.join(ORACLE, "liboracle_hrf_san.so"),
        "LD_PRELOAD": asan,
        "ASAN_OPTIONS": "detect_leaks=0:verify_asan_link_order=0:abort_on_error=1",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
        "OMP_NUM_THREADS": "4",
    })
    files = [os.path.join(REPO, "tests", f) for f in ("test_oracle_pinning.py", "test_golden.py")]
    res = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                          *files], cwd=REPO, env=env, capture_output=True, text=True)
    tail = (res.stdout + res.stderr)[-4000:]
    assert res.returncode == 0, tail
    assert "AddressSanitizer" not in tail and "runtime error" not in tail, tail
