"""Drop-in for the reference package ``cuda_prop`` (cuda_prop/__init__.py):
the names ``model.py:37`` imports, backed by the gfx950 HIP library."""
from .python_function import (  # noqa: F401
    BandlimitedPropagation,
    BandlimitedPropagationFunction,
    MultiPlanePropagationFunction,
    compute_bmm_cuda,
    cuda_module,
    element_wise_multiplication_cuda,
    multiplane_propagation,
    sum_last_dim_cuda,
)
