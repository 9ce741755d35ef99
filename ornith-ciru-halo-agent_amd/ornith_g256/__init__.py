"""MI355X-native Ornith G256 quantized-MoE hot path.

Host package mirroring the reference plugin's native boundary
(plugin-site/ornith_g256/native.py) on top of one gfx950 HIP library
(lib/libornith_g256_mi355x.so, sources in ../csrc)."""
from . import native  # noqa: F401

__all__ = ['native']
