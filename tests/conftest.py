import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.complex128 if np.iscomplexobj(a) or np.iscomplexobj(b) else np.float64)
    b = np.asarray(b, dtype=a.dtype)
    den = np.linalg.norm(b.ravel())
    num = np.linalg.norm((a - b).ravel())
    if den == 0:
        return float(num)
    return float(num / den)


def oracle_inputs(sc):
    """Scene (package generator) -> oracle Gaussians / Camera."""
    from oracle import oracle as O

    g = O.Gaussians(sc.cam_means, sc.z, sc.quats, sc.scales, sc.colours, sc.phase, sc.opac,
                    sc.pprobs)
    cam = O.Camera(sc.fx, sc.fy, sc.px, sc.py, sc.view, sc.spec.width, sc.spec.height, 1.0,
                   1000.0)
    return g, cam


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle as O

    O.lib()
    return O


def gpu_available():
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def hrf():
    if not gpu_available():
        pytest.skip("no GPU")
    import complex_valued_holographic_radiance_fields_amd as pkg

    return pkg
