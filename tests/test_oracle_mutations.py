"""The pins of the oracle's non-derivative gradient formulas detect one-term
mistakes: each case copies hrf_oracle.c to a temporary directory, plants one
mistake in the copy (a dropped term, a transposed factor, a flipped sign),
builds it, and reruns the pin tests against that build in a child
interpreter (HRF_ORACLE_LIB), which must fail.  The unmodified copy must
pass, so a failure is the mistake's doing.  Everything here runs on the
CPU; nothing under oracle/ is modified."""
import os
import shutil
import subprocess
import sys

import pytest

from conftest import REPO

SRC = os.path.join(REPO, "oracle", "hrf_oracle.c")
CFLAGS = ["-O2", "-fPIC", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-shared"]

PINS = ("test_quaternion_gradient_is_derivative_of_hadamard_form or "
        "test_scale_gradient_is_derivative_at_conjugate_rotation or "
        "test_cov2d_gradient_map_diagonal_closed_form or test_cov2d_gradient_map_in_conic_form")

MUTANTS = {
    # Hadamard sum with one of its two products dropped (backward.cu:161-187)
    "quat_term_dropped": ("gr += Gm[i][j] * (Xr[j][i] * SR[i][j] + SR[j][i] * Xr[i][j]);",
                          "gr += Gm[i][j] * (Xr[j][i] * SR[i][j]);"),
    # R^T G R replaced by (R^T)^T G R^T: the scale gradient at q instead of q_bar
    "scale_transposed": ("glm_mul(T1, R, temp);",
                         "{ float Rt[3][3]; for (int c = 0; c < 3; ++c) for (int rr = 0; rr < 3; "
                         "++rr) Rt[c][rr] = R[rr][c]; glm_mul(T1, Rt, temp); }"),
    # the conic_z term of the xx entry dropped (backward_splat.cu:285-286)
    "cov_xx_term_dropped": ("dL_dconic_z * (-cy * det_inv * det_inv) * (-cy);",
                            "0.0f;"),
    # the sign of the conic_y term of the xy entry flipped (backward_splat.cu:287-289)
    "cov_xy_sign": ("dL_dconic_y * (-det_inv) +", "dL_dconic_y * (det_inv) +"),
}


def _run_pins(tmp, name, source):
    cdir = os.path.join(tmp, name)
    os.makedirs(cdir, exist_ok=True)
    c = os.path.join(cdir, "hrf_oracle.c")
    with open(c, "w") as f:
        f.write(source)
    so = os.path.join(cdir, "liboracle.so")
    subprocess.run(["gcc", *CFLAGS, "-o", so, c, "-lm"], check=True, capture_output=True)
    env = dict(os.environ, HRF_ORACLE_LIB=so, OMP_NUM_THREADS="4")
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                          os.path.join(REPO, "tests", "test_oracle_pinning.py"), "-k", PINS],
                         cwd=REPO, env=env, capture_output=True, text=True)
    return res.returncode, (res.stdout + res.stderr)[-3000:]


@pytest.mark.timeout(600)
def test_pins_fail_on_planted_mistakes(tmp_path):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    src = open(SRC).read()
    rc, out = _run_pins(str(tmp_path), "unmodified", src)
    assert rc == 0, out
    for name, (old, new) in MUTANTS.items():
        assert src.count(old) == 1, (name, "mutation site not found exactly once")
        rc, out = _run_pins(str(tmp_path), name, src.replace(old, new))
        assert rc != 0, f"mutant {name} passed the pins:\n{out}"
        assert "failed" in out, out
