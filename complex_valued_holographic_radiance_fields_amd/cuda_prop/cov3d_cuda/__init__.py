"""Drop-in for the reference package ``cuda_prop.cov3d_cuda``."""
