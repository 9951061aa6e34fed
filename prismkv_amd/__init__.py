"""prismkv_amd -- MI355X-native (gfx950) kernels for PrismKV's routed decode path.

`Native8B` is the drop-in for the reference's `prismkv.native8b.Native8B`;
the HIP kernels behind it live in `csrc/` and are reached through the C ABI
declared in `include/prismkv_hip.h`.
"""
from .native8b import FeatureIndex, Native8B, compile_hip, tile_moments, untile_moments
from ._lib import load as load_library

__all__ = ["FeatureIndex", "Native8B", "compile_hip", "load_library", "tile_moments", "untile_moments"]
