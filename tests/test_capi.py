"""CPU checks of the C ABI library: it loads, exports every entry point that
include/hrf.h declares, and its host-only sizing functions behave (no GPU
calls are made here)."""
import ctypes
import os
import re

import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "hrf.h")
LIB = os.path.join(REPO, "complex_valued_holographic_radiance_fields_amd", "lib", "libhrf.so")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"\b(hrf_[a-z0-9_]+)\s*\(", src)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libhrf.so is not built (run __graft_entry__.build())")
    return ctypes.CDLL(LIB)


def test_header_lists_entry_points():
    names = declared_functions()
    assert "hrf_raster_forward_prepare" in names
    assert "hrf_asm_multiplane_forward" in names
    assert len(names) >= 15


def test_all_declared_symbols_exported(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    from complex_valued_holographic_radiance_fields_amd import _lib

    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_workspace_sizes_monotone(lib):
    f = lib.hrf_raster_geom_workspace_size
    f.restype = ctypes.c_size_t
    f.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32]
    a, b = f(1000, 3, 3), f(1_000_000, 3, 3)
    assert 0 < a < b
    assert b < 1_000_000 * 200  # ~O(100 B) per Gaussian
    g = lib.hrf_raster_binning_workspace_size
    g.restype = ctypes.c_size_t
    g.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32]
    assert g(10, 64, 64) < g(10_000_000, 64, 64)
    h = lib.hrf_asm_workspace_size
    h.restype = ctypes.c_size_t
    h.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
    M = 1600
    assert h(3, 3, 800) >= (9 + 3) * M * M * 8


def test_version_and_error_strings(lib):
    lib.hrf_version.restype = ctypes.c_char_p
    assert b"gfx950" in lib.hrf_version()
    lib.hrf_last_error.restype = ctypes.c_char_p
    assert isinstance(lib.hrf_last_error(), bytes)


def test_invalid_arguments_rejected_without_gpu(lib):
    """Argument validation happens before any HIP call."""
    from complex_valued_holographic_radiance_fields_amd import _lib as L

    f = lib.hrf_raster_forward_prepare
    f.restype = ctypes.c_int
    f.argtypes = L.SIGNATURES["hrf_raster_forward_prepare"][1]
    g = L.HrfGaussians(None, None, None, None, None, None, None, None, 10, 4, 1)
    c = L.HrfCamera(1.0, 1.0, 0.0, 0.0, None, 16, 16, 1.0, 1000.0)
    k = ctypes.c_int64(0)
    v = ctypes.c_int64(0)
    st = f(ctypes.byref(g), ctypes.byref(c), None, 0, None, ctypes.byref(k), ctypes.byref(v))
    assert st == 1
    lib.hrf_last_error.restype = ctypes.c_char_p
    assert b"channels" in lib.hrf_last_error()


def test_reference_import_statements_resolve():
    """The names model.py:16-19 and :37 import exist in the drop-in modules
    (a missing one makes the reference fall back to its Python path)."""
    from complex_valued_holographic_radiance_fields_amd.cuda_prop import (  # noqa: F401
        BandlimitedPropagation, compute_bmm_cuda, element_wise_multiplication_cuda,
        sum_last_dim_cuda)
    from complex_valued_holographic_radiance_fields_amd.cuda_prop.cov3d_cuda.python_import \
        import (compute_cov2d_cuda, compute_cov3d_cuda, compute_jacobian_cuda,  # noqa: F401
                compute_means2d_cuda, invert_cov2d_cuda, splat_tile_cuda)


def test_geometry_operators_reject_host_tensors():
    """As the reference's operators: ValueError for non-GPU inputs, raised
    before any HIP call."""
    import torch
    from complex_valued_holographic_radiance_fields_amd.cuda_prop.cov3d_cuda import \
        python_import as pi

    with pytest.raises(ValueError):
        pi.compute_cov3d_cuda(torch.zeros(3, 4), torch.ones(3, 3))
    with pytest.raises(ValueError):
        pi.invert_cov2d_cuda(torch.eye(2).expand(3, 2, 2))
    with pytest.raises(ValueError):
        pi.compute_means2d_cuda(torch.ones(3, 3), 1.0, 1.0, 0.0, 0.0, 1.0, 100.0)
