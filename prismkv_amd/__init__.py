"""prismkv_amd -- MI355X-native (gfx950) kernels for PrismKV's routed decode path.

`Native8B` is the drop-in for the reference's `prismkv.native8b.Native8B`;
the HIP kernels behind it live in `csrc/` and are reached through the C ABI
declared in `include/prismkv_hip.h`.  `prismkv_amd.weights` reads and writes
the reference's encoder bundles; `prismkv_amd.hf.HFNative` is the Hugging
Face decode backend over `Native8B` (imports transformers when used).
"""
from .native8b import FeatureIndex, Native8B, compile_hip, set_spin_limit, tile_moments, untile_moments
from ._lib import load as load_library
from .weights import Encoder, SharedSAE, load_encoders, save_encoders

__all__ = ["Encoder", "FeatureIndex", "Native8B", "SharedSAE", "compile_hip", "load_encoders", "load_library",
           "save_encoders", "set_spin_limit", "tile_moments", "untile_moments"]
