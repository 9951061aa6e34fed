"""ctypes binding of libprismkv_hip.so (declarations in include/prismkv_hip.h).

Argument convention of the reference binding (src/prismkv/native8b.py:46-51):
device pointers as uint64, then integer sizes, then the stream; integer return
code, 0 on success.  A nonzero code raises RuntimeError exactly as the
reference's `Native8B.call` does (src/prismkv/native8b.py:76-80).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

DEFAULT_LIBRARY = Path(__file__).resolve().with_name("libprismkv_hip.so")

_U64, _I32, _I64, _SZ = ctypes.c_uint64, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t

# name -> (argument types without the trailing stream, has_stream, restype)
SIGNATURES = {
    # reference-compatible symbols
    "pack": ([_U64] * 2, True, _I32),
    "build_bits": ([_U64] * 3 + [_I32] * 2, True, _I32),
    "fused_norm_top": ([_U64] * 6, True, _I32),
    "launch_union_warp": ([_U64] * 7 + [_I32] * 3, True, _I32),
    "attention_tuned": ([_U64] * 7 + [_I32] * 6, True, _I32),
    # MI355X-native symbols
    "prismkv_route_work_bytes": ([_I32], False, _SZ),
    "prismkv_route": ([_U64] * 7 + [_I32, _SZ], True, _I32),
    "prismkv_route_single": ([_U64] * 7 + [_I32, _SZ], True, _I32),
    "prismkv_route_union": ([_U64] * 10 + [_I32, _I32, _I32, _I64, _I64, _SZ], True, _I32),
    "prismkv_union_work_bytes": ([_I32, _I32], False, _SZ),
    "prismkv_union": ([_U64] * 6 + [_I32, _I32, _I64, _I64, _SZ], True, _I32),
    "prismkv_build_bits": ([_U64] * 3 + [_I32, _I64, _I64], True, _I32),
    "prismkv_attend_work_bytes": ([_I32, _I32], False, _SZ),
    "prismkv_attend": ([_U64] * 7 + [_I32, _I32, _I32, _I64, _I64, _I64, _I32, _SZ], True, _I32),
    "prismkv_decode_work_bytes": ([_I32, _I32], False, _SZ),
    "prismkv_decode": ([_U64] * 13 + [_I32, _I32, _I32, _I32, _I64, _I64, _I64, _I64, _SZ], True, _I32),
    "prismkv_union_attend": ([_U64] * 10 + [_I32, _I32, _I32, _I32, _I64, _I64, _I64, _I64, _SZ], True, _I32),
    "prismkv_decode_tail": ([_U64] * 14 + [_I32, _I32, _I32, _I32, _I64, _I64, _I64, _I64, _SZ], True, _I32),
    "prismkv_union_attend_tail": ([_U64] * 11 + [_I32, _I32, _I32, _I32, _I64, _I64, _I64, _I64, _SZ], True,
                                  _I32),
    "prismkv_decode_capped": ([_U64] * 13 + [_I32, _I32, _I32, _I32, _I64, _I64, _I64, _I64, _I64, _SZ], True,
                              _I32),
    "prismkv_decode_capped_tail": ([_U64] * 14 + [_I32, _I32, _I32, _I32, _I64, _I64, _I64, _I64, _I64, _SZ],
                                   True, _I32),
    "prismkv_select_cap": ([_U64] * 5 + [_I32, _I32, _I64, _I64], True, _I32),
    "prismkv_update_work_bytes": ([_I32, _I32], False, _SZ),
    "prismkv_update_act_offset": ([_I32], False, _SZ),
    "prismkv_update": ([_U64] * 9 + [_I32] * 4 + [_I64, _I64, _SZ], True, _I32),
    "prismkv_build_work_bytes": ([_I32, _I32], False, _SZ),
    "prismkv_build": ([_U64] * 9 + [_I32] * 5 + [_I64, _I64, _SZ], True, _I32),
    "prismkv_route_scores": ([_U64] * 8 + [_I32, _SZ], True, _I32),
    "prismkv_topk_work_bytes": ([], False, _SZ),
    "prismkv_topk": ([_U64] * 4 + [_I32, _I64, _SZ], True, _I32),
    "prismkv_summarize_work_bytes": ([_I32], False, _SZ),
    "prismkv_summarize": ([_U64] * 6 + [_I32, _I32, _I32, _I64, _I64, _SZ], True, _I32),
    "prismkv_route_qact_work_bytes": ([_I32], False, _SZ),
    "prismkv_route_qact": ([_U64] * 10 + [_I32, _SZ], True, _I32),
    "prismkv_build_f32": ([_U64] * 9 + [_I32] * 5 + [_I64, _I64, _SZ], True, _I32),
    "prismkv_update_f32": ([_U64] * 9 + [_I32] * 4 + [_I64, _I64, _SZ], True, _I32),
    "prismkv_summarize_f32": ([_U64] * 6 + [_I32, _I32, _I32, _I64, _I64, _SZ], True, _I32),
    "prismkv_route_scores_f32": ([_U64] * 8 + [_I32, _SZ], True, _I32),
    "prismkv_route_qact_f32": ([_U64] * 10 + [_I32, _SZ], True, _I32),
    "prismkv_attend_f32": ([_U64] * 7 + [_I32, _I32, _I32, _I64, _I64, _I64, _I32, _SZ], True, _I32),
    "prismkv_union_n": ([_U64] * 6 + [_I32, _I32, _I64, _I64, _I32, _SZ], True, _I32),
    "prismkv_select_cap_n": ([_U64] * 5 + [_I32, _I32, _I64, _I64, _I32], True, _I32),
    # error handling of the bounded inter-workgroup waits
    "prismkv_set_spin_limit": ([_I32], False, _I32),
    "prismkv_get_spin_limit": ([], False, _I32),
    "prismkv_mapped_pointer": ([_U64], False, _U64),
    # the allocation-free decode (workspace in the library's own device array)
    "prismkv_scratch_bytes": ([], False, _SZ),
    "prismkv_decode_noalloc": ([_U64] * 13 + [_I32] * 4 + [_I64] * 4, True, _I32),
}

_loaded: dict[str, "Library"] = {}


class Library:
    """A loaded libprismkv_hip.so with typed entry points."""

    def __init__(self, path=None):
        path = Path(path or DEFAULT_LIBRARY).resolve()
        if not path.exists():
            raise RuntimeError(f"{path.name} is not built at {path}; run `python -c \"import __graft_entry__ as g; "
                               f"g.build()\"` (hipcc --offload-arch=gfx950) first")
        self.path = path
        self.cdll = ctypes.CDLL(str(path))
        self.missing = []
        for name, (args, stream, res) in SIGNATURES.items():
            fn = getattr(self.cdll, name, None)
            if fn is None:
                self.missing.append(name)
                continue
            fn.argtypes = list(args) + ([_U64] if stream else [])
            fn.restype = res

    def has(self, name: str) -> bool:
        return hasattr(self.cdll, name)

    def call(self, name: str, *args, stream: int):
        code = getattr(self.cdll, name)(*args, stream)
        if code:
            raise RuntimeError(f"{name}: device launch error {code}")

    def query(self, name: str, *args) -> int:
        return int(getattr(self.cdll, name)(*args))


def nbytes(t) -> int:
    """Size in bytes of a workspace tensor: the `work_bytes` argument that
    accompanies its pointer."""
    return t.numel() * t.element_size()


def load(path=None) -> Library:
    key = str(Path(path or DEFAULT_LIBRARY).resolve())
    lib = _loaded.get(key)
    if lib is None:
        lib = _loaded[key] = Library(key)
    return lib
