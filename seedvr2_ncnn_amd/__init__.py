"""seedvr2_ncnn_amd: SeedVR2's DiT window-attention hot path on MI355X (gfx950).

The product is native code:
  lib/libseedvr2_hip.so     gfx950 kernels behind the C-ABI of include/seedvr2_hip.h
  lib/libseedvr2_layers.so  the ncnn-surface C++ layers AdaptiveWindowAttention and
                            SharedLinear calling that C-ABI
This Python package only builds them (build.py) and binds the C-ABI for tests
and benchmarks (capi.py).
"""
from . import capi  # noqa: F401

__all__ = ["capi"]
