"""MI355X-native (gfx950) complex-valued wave rasterizer and band-limited ASM
propagator — a drop-in for the hot path of Complex-Valued Holographic
Radiance Fields.

Drop-in entry points (same names and signatures as the reference):
  complex_valued_holographic_radiance_fields_amd.cuda_prop.cov3d_cuda.python_import
      .splat_tile_cuda / .SplatTileCuda / .Rasterizer
  complex_valued_holographic_radiance_fields_amd.cuda_prop
      .BandlimitedPropagation / .BandlimitedPropagationFunction / .cuda_module

The kernels live in lib/libhrf.so (C ABI: include/hrf.h), built with
``build.build_library()``; importing this package loads it and raises if it
is missing.
"""
from . import _lib

_lib.load()

from . import propagation, rasterizer  # noqa: E402,F401

__all__ = ["propagation", "rasterizer"]
