"""CPU checks of the C ABI: the library loads, exports every entry point the
header declares, and rejects invalid arguments on the host with the reference
error codes (-1 size/range, -2 mode) before enqueuing anything."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "prismkv_hip.h"


@pytest.fixture(scope="module")
def lib():
    from prismkv_amd import _lib
    if not _lib.DEFAULT_LIBRARY.exists():
        from prismkv_amd.build import build_inplace
        build_inplace()
    return _lib.load()


def declared_symbols():
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:int|size_t|uint64_t)\s+(\w+)\s*\(", text, flags=re.M)


def test_header_declares_reference_symbols():
    names = declared_symbols()
    # src/prismkv/native8b.py:46-48: the five symbols a reference-shaped binding binds
    for ref in ["pack", "build_bits", "fused_norm_top", "launch_union_warp", "attention_tuned"]:
        assert ref in names
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol(lib):
    names = declared_symbols()
    missing = [n for n in names if not lib.has(n)]
    assert not missing, missing
    from prismkv_amd import _lib
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def test_library_is_gfx950():
    from prismkv_amd import _lib
    data = _lib.DEFAULT_LIBRARY.read_bytes() if _lib.DEFAULT_LIBRARY.exists() else b""
    assert b"gfx950" in data


def test_work_size_queries(lib):
    assert lib.query("prismkv_route_work_bytes", 8) >= 8 * 4 * 3008 * 4
    assert lib.query("prismkv_route_work_bytes", 0) == 0
    assert lib.query("prismkv_union_work_bytes", 8, 65536) > 8
    assert lib.query("prismkv_attend_work_bytes", 8, 64) >= 8 * 4 * 64 * 130 * 4
    # the update workspace holds the block's dense activations [G][N][3000] f32
    assert lib.query("prismkv_update_work_bytes", 8, 4096) >= 8 * 4096 * 3000 * 4
    assert lib.query("prismkv_update_work_bytes", 8, 4097) == 0
    assert lib.query("prismkv_update_work_bytes", 0, 16) == 0
    # the build workspace holds one batch's activations [batch][H][3000] f32
    assert lib.query("prismkv_build_work_bytes", 8, 65536) >= 8 * 65536 * 3000 * 4
    assert lib.query("prismkv_build_work_bytes", 1, 1 << 20) >= (1 << 20) * 3000 * 4
    assert lib.query("prismkv_build_work_bytes", 1, (1 << 20) + 1) == 0
    assert lib.query("prismkv_build_work_bytes", 0, 16) == 0
    # the activations follow regions whose offsets depend on the group count
    # only; after them the compact candidate list: at least 2^19 entries of
    # 8 bytes per group, 16 per key for a build's long blocks
    at = lib.query("prismkv_update_act_offset", 8)
    assert at > 0 and at % 256 == 0 and lib.query("prismkv_update_act_offset", 0) == 0
    for n in (1, 37, 4096):
        act = (8 * n * 3000 * 4 + 255) // 256 * 256
        assert lib.query("prismkv_update_work_bytes", 8, n) - at >= act + 8 * (1 << 19) * 8
    assert lib.query("prismkv_build_work_bytes", 3, 65536) - lib.query("prismkv_update_act_offset", 3) >= \
        3 * 65536 * 3000 * 4 + 3 * 16 * 65536 * 8


def call_raw(lib, name, *args):
    return getattr(lib.cdll, name)(*args, 0)


def test_compat_error_codes(lib):
    # kernels/ppu_8b/union.cu:40,47: U in [1,8], H in [1,131072], mode in {0,1,2}
    for U, H, mode, code in [(0, 100, 2, -1), (9, 100, 2, -1), (8, 0, 2, -1), (8, 131073, 2, -1),
                             (8, 100, 3, -2), (8, 100, -1, -2)]:
        assert call_raw(lib, "launch_union_warp", *[0] * 7, U, H, mode) == code
    # kernels/ppu_8b/av_tuned.cu:63,65
    H, T = 100, 5
    good = (H + T) * 128
    for S, h, t, ks, vs, mode, code in [(0, H, T, good, good, 0, -1), (129, H, T, good, good, 0, -1),
                                         (64, 0, T, good, good, 0, -1), (64, H, -1, good, good, 0, -1),
                                         (64, H, T, good - 1, good, 0, -1), (64, H, T, good, good - 1, 0, -1),
                                         (64, H, T, good, good, 3, -2)]:
        assert call_raw(lib, "attention_tuned", *[0] * 7, h, t, ks, vs, S, mode) == code


BIG = 1 << 40  # a work_bytes that passes the workspace-size check, so the other checks decide


def test_native_error_codes(lib):
    assert call_raw(lib, "prismkv_route", *[0] * 7, 8, BIG) == -1          # null pointers
    assert call_raw(lib, "prismkv_route", *[1] * 7, 0, BIG) == -1          # no groups
    assert call_raw(lib, "prismkv_route_single", *[0] * 7, 8, BIG) == -1   # null pointers
    assert call_raw(lib, "prismkv_route_single", *[1] * 7, 0, BIG) == -1   # no groups
    ua = (8, 100, 4, 100, 4, 104 * 128, 104 * 128, 100)
    assert call_raw(lib, "prismkv_union_attend", *[0] * 10, *ua, BIG) == -1
    assert call_raw(lib, "prismkv_union_attend", *[1] * 10, 8, 0, *ua[2:], BIG) == -1
    assert call_raw(lib, "prismkv_union_attend", *[1] * 10, *ua[:5], 103 * 128, *ua[6:], BIG) == -1
    assert call_raw(lib, "prismkv_union", *[1] * 6, 8, 0, 1, 1, BIG) == -1  # H < 1
    assert call_raw(lib, "prismkv_union", *[1] * 6, 8, 100, 3, 100, BIG) == -1  # row_words too small
    assert call_raw(lib, "prismkv_union", *[1] * 6, 8, 100, 4, 99, BIG) == -1   # ids stride too small
    assert call_raw(lib, "prismkv_attend", *[1] * 7, 8, 10, 2, 12 * 128, 12 * 128, 10, 0, BIG) == -1  # splits
    assert call_raw(lib, "prismkv_attend", *[1] * 7, 8, 10, 2, 11 * 128, 12 * 128, 10, 4, BIG) == -1  # ks
    assert call_raw(lib, "prismkv_attend_f32", *[16] * 7, 8, 10, 2, 11 * 128, 12 * 128, 10, 4, BIG) == -1  # ks
    assert call_raw(lib, "prismkv_attend_f32", 20, *[16] * 6, 8, 10, 2, 12 * 128, 12 * 128, 10, 4, BIG) == -1  # q
    assert call_raw(lib, "prismkv_attend_f32", *[16] * 7, 8, 10, 2, 12 * 128 + 1, 12 * 128, 10, 4, BIG) == -1  # ks
    assert call_raw(lib, "prismkv_build_f32", *[16] * 9, 8, 8, 100, 8, 0, 100 * 128 + 2, 4, BIG) == -1  # K stride
    assert call_raw(lib, "prismkv_build_f32", *[0] * 9, 8, 8, 100, 8, 0, 100 * 128, 4, BIG) == -1  # null pointers
    assert call_raw(lib, "prismkv_route_scores_f32", *[16] * 7, 0, 8, BIG) == -1  # no score vector
    # prismkv_update(k, W, b, center, scale, bits, counts, moments, work, groups, H, N, key_mean, ks, row_words,
    # work_bytes)
    good = (100 + 64) * 128
    for G, H, N, km, ks, rw in [(8, 100, 0, 8, good, 8), (8, 100, 4097, 8, 4197 * 128, 132), (8, 100, 64, 0, good, 8),
                                (8, 100, 64, 3001, good, 8), (8, 100, 64, 8, good - 1, 8), (8, 100, 64, 8, good, 5),
                                (0, 100, 64, 8, good, 8), (8, -1, 64, 8, good, 8)]:
        assert call_raw(lib, "prismkv_update", *[1] * 9, G, H, N, km, ks, rw, BIG) == -1, (G, H, N, km, ks, rw)
    assert call_raw(lib, "prismkv_update", *[0] * 9, 8, 100, 64, 8, good, 8, BIG) == -1  # null pointers
    # prismkv_build(k, W, b, center, scale, bits, counts, moments, work, groups, batch, H, key_mean, flags, ks,
    # row_words, work_bytes): 16-byte aligned fake pointers, so only the sizes decide
    good = 100 * 128
    for G, B, H, km, fl, ks, rw in [(0, 1, 100, 8, 0, good, 4), (8, 0, 100, 8, 0, good, 4), (8, 9, 100, 8, 0, good, 4),
                                    (8, 8, 0, 8, 0, good, 4), (8, 8, (1 << 20) + 1, 8, 0, 1 << 28, 32772),
                                    (8, 8, 100, 0, 0, good, 4), (8, 8, 100, 3001, 0, good, 4),
                                    (8, 8, 100, 8, 0, good - 128, 4), (8, 8, 100, 8, 0, good, 3),
                                    (8, 8, 100, 8, 0, good, 5)]:
        assert call_raw(lib, "prismkv_build", *[16] * 9, G, B, H, km, fl, ks, rw, BIG) == -1, (G, B, H, km, fl, ks,
                                                                                               rw)
    assert call_raw(lib, "prismkv_build", *[16] * 9, 8, 8, 100, 8, 2, good, 4, BIG) == -2  # unknown flag
    assert call_raw(lib, "prismkv_build", *[0] * 9, 8, 8, 100, 8, 0, good, 4, BIG) == -1   # null pointers
    assert call_raw(lib, "prismkv_build", *[18] + [16] * 8, 8, 8, 100, 8, 0, good, 4, BIG) == -1  # misaligned K
    assert call_raw(lib, "prismkv_build", 16, 20, *[16] * 7, 8, 8, 100, 8, 0, good, 4, BIG) == -1  # misaligned W
    assert call_raw(lib, "prismkv_build", 16, 16, 24, *[16] * 6, 8, 8, 100, 8, 0, good, 4, BIG) == -1  # misaligned b
    good = (100 + 64) * 128
    assert call_raw(lib, "prismkv_update", 16, 20, *[16] * 7, 8, 100, 64, 8, good, 8, BIG) == -1  # misaligned W
    assert call_raw(lib, "prismkv_update", 16, 16, 24, *[16] * 6, 8, 100, 64, 8, good, 8, BIG) == -1  # misaligned b
    # prismkv_decode(13 buffers, groups, H, T, capacity, row_words, ks, vs, ids_stride, work_bytes, stream): K/V
    # rows are addressed by 32-bit byte offsets, so (H + T) x 256 must stay below 2^31
    big = (100 + (1 << 23)) * 128
    assert call_raw(lib, "prismkv_decode", *[16] * 13, 8, 100, 1 << 23, 100, 4, big, big, 100, BIG) == -1
    # prismkv_decode_tail(13 buffers, tail, groups, H, max_tail, capacity, row_words, ks, vs, ids_stride,
    # work_bytes)
    ok = (100 + 8) * 128
    assert call_raw(lib, "prismkv_decode_tail", *[16] * 13, 0, 8, 100, 8, 100, 4, ok, ok, 100, BIG) == -1  # no word
    assert call_raw(lib, "prismkv_decode_tail", *[16] * 13, 18, 8, 100, 8, 100, 4, ok, ok, 100, BIG) == -1  # misal.
    assert call_raw(lib, "prismkv_decode_tail", *[16] * 14, 8, 100, -1, 100, 4, ok, ok, 100, BIG) == -1  # bound < 0
    assert call_raw(lib, "prismkv_decode_tail", *[16] * 14, 8, 100, 9, 100, 4, ok, ok, 100, BIG) == -1  # K short


# Every entry point that takes a workspace, with valid sizes and 16-byte
# aligned fake pointers: name -> (arguments before work_bytes, the
# *_work_bytes query and its arguments).  With one byte less than the query
# the call is refused with -1 before anything is enqueued; with the queried
# size it passes the host checks and (no GPU here) fails at the launch with
# the runtime's error, or, for the entry points whose groups wait on each
# other, at the residency check (-1), which they make after the size check.
H, T, KS = 1000, 24, (1000 + 24) * 128
WORK_CASES = {
    "prismkv_route": ((*[16] * 7, 8), ("prismkv_route_work_bytes", 8)),
    "prismkv_route_scores": ((*[16] * 8, 8), ("prismkv_route_work_bytes", 8)),
    "prismkv_route_qact": ((*[16] * 10, 8), ("prismkv_route_qact_work_bytes", 8)),
    "prismkv_union": ((*[16] * 6, 8, H, 32, H), ("prismkv_union_work_bytes", 8, H)),
    "prismkv_union_n": ((*[16] * 6, 8, H, 32, H, 64), ("prismkv_union_work_bytes", 8, H)),
    "prismkv_attend": ((*[16] * 7, 8, H, T, KS, KS, H, 32), ("prismkv_attend_work_bytes", 8, 32)),
    "prismkv_update": ((*[16] * 9, 8, H, T, 8, KS, 32), ("prismkv_update_work_bytes", 8, T)),
    "prismkv_build": ((*[16] * 9, 8, 4, H, 8, 1, KS, 32), ("prismkv_build_work_bytes", 4, H)),
    "prismkv_topk": ((*[16] * 4, 100, 800), ("prismkv_topk_work_bytes",)),
    "prismkv_summarize": ((*[16] * 6, 8, H, 1, KS, 32), ("prismkv_summarize_work_bytes", 8)),
    "prismkv_route_scores_f32": ((*[16] * 8, 8), ("prismkv_route_work_bytes", 8)),
    "prismkv_route_qact_f32": ((*[16] * 10, 8), ("prismkv_route_qact_work_bytes", 8)),
    "prismkv_attend_f32": ((*[16] * 7, 8, H, T, KS, KS, H, 32), ("prismkv_attend_work_bytes", 8, 32)),
    "prismkv_update_f32": ((*[16] * 9, 8, H, T, 8, KS, 32), ("prismkv_update_work_bytes", 8, T)),
    "prismkv_build_f32": ((*[16] * 9, 8, 4, H, 8, 1, KS, 32), ("prismkv_build_work_bytes", 4, H)),
    "prismkv_summarize_f32": ((*[16] * 6, 8, H, 1, KS, 32), ("prismkv_summarize_work_bytes", 8)),
    "prismkv_route_single": ((*[16] * 7, 8), ("prismkv_decode_work_bytes", 8, H)),
    "prismkv_route_union": ((*[16] * 10, 8, H, H, 32, H), ("prismkv_decode_work_bytes", 8, H)),
    "prismkv_decode": ((*[16] * 13, 8, H, T, H, 32, KS, KS, H), ("prismkv_decode_work_bytes", 8, H)),
    "prismkv_decode_tail": ((*[16] * 14, 8, H, T, H, 32, KS, KS, H), ("prismkv_decode_work_bytes", 8, H)),
    "prismkv_decode_capped": ((*[16] * 13, 8, H, T, H, 62, 32, KS, KS, H), ("prismkv_decode_work_bytes", 8, H)),
    "prismkv_decode_capped_tail": ((*[16] * 14, 8, H, T, H, 62, 32, KS, KS, H),
                                   ("prismkv_decode_work_bytes", 8, H)),
    "prismkv_union_attend": ((*[16] * 10, 8, H, T, H, 32, KS, KS, H), ("prismkv_decode_work_bytes", 8, H)),
    "prismkv_union_attend_tail": ((*[16] * 11, 8, H, T, H, 32, KS, KS, H), ("prismkv_decode_work_bytes", 8, H)),
}
WAITING = {"prismkv_route_single", "prismkv_route_union", "prismkv_decode", "prismkv_decode_tail", "prismkv_decode_capped",
           "prismkv_decode_capped_tail", "prismkv_union_attend", "prismkv_union_attend_tail"}


def test_every_work_entry_point_is_covered(lib):
    from prismkv_amd import _lib
    takes_work = {name for name in _lib.SIGNATURES if name.startswith("prismkv_") and
                  re.search(r"\buint64_t work\b", _declaration(name))}
    assert takes_work == set(WORK_CASES), takes_work ^ set(WORK_CASES)


def _declaration(name):
    text = HEADER.read_text()
    m = re.search(r"^\s*(?:int|size_t|uint64_t)\s+" + name + r"\s*\(([^;]*)\);", text, flags=re.M)
    assert m, name
    return m.group(1)


@pytest.mark.parametrize("name", sorted(WORK_CASES))
def test_undersized_workspace_is_refused(lib, name):
    args, (query, *qargs) = WORK_CASES[name]
    assert "size_t work_bytes, uint64_t stream" in " ".join(_declaration(name).split())
    need = lib.query(query, *qargs)
    assert need > 0
    assert call_raw(lib, name, *args, need - 1) == -1
    assert call_raw(lib, name, *args, 0) == -1
    rc = call_raw(lib, name, *args, need)
    if name in WAITING:
        assert rc == -1  # no device: the residency check, made after the size check
    else:
        assert rc not in (0, -1, -2), rc  # past every host check, refused by the runtime (no device)


def test_native8b_host_validation_without_gpu():
    import torch
    from prismkv_amd import FeatureIndex, Native8B
    idx = FeatureIndex(4, torch.zeros(128), torch.zeros(3000, dtype=torch.long), torch.zeros(3000, 128),
                       torch.zeros(3000, 128), [torch.zeros(0, dtype=torch.long)] * 3000)
    with pytest.raises(ValueError, match="8 KV groups"):
        Native8B([idx] * 7)
    with pytest.raises(ValueError, match="device tensor"):
        Native8B([idx] * 8)


def test_spin_limit_is_host_settable(lib):
    from prismkv_amd import set_spin_limit
    default = lib.query("prismkv_get_spin_limit")
    assert default == 1 << 20
    assert set_spin_limit(12345) == default
    try:
        assert lib.query("prismkv_get_spin_limit") == 12345
        assert lib.query("prismkv_set_spin_limit", -1) == -1  # rejected, unchanged
        assert lib.query("prismkv_get_spin_limit") == 12345
    finally:
        assert set_spin_limit(default) == 12345
    with pytest.raises(ValueError):
        set_spin_limit(-1)


def test_mapped_pointer_rejects_null(lib):
    assert lib.query("prismkv_mapped_pointer", 0) == 0
