"""The allocation-free decode entry point (prismkv_decode_noalloc) against
prismkv_decode.

prismkv_decode_noalloc takes the decode workspace from the library's own
file-scope device array instead of a caller buffer; everything else is the
same launch.  Two calls in a row (the second with a smaller history and
tail, so the array still holds the first call's layout) must reproduce
prismkv_decode's outputs bit for bit: selection, ids, count and out.
"""
import numpy as np
import pytest
import torch

from oracle import cases
from tests.gpu_util import log, operator

pytestmark = pytest.mark.gpu


def _noalloc(op, q, k, v, groups=8, history=None):
    """prismkv_decode_noalloc into fresh output buffers; returns them and the error word."""
    history = op.history if history is None else history
    dev = q.device
    out = dict(features=torch.zeros(groups, 16, dtype=torch.int64, device=dev),
               valid=torch.zeros(groups, 16, device=dev), raw=torch.zeros(groups, dtype=torch.int32, device=dev),
               ids=torch.zeros(groups, op.capacity, dtype=torch.int32, device=dev),
               count=torch.zeros(groups, dtype=torch.int32, device=dev),
               out=torch.zeros(groups, 4, 128, dtype=torch.bfloat16, device=dev),
               err=torch.zeros(1, dtype=torch.int32, device=dev))
    rc = op.lib.cdll.prismkv_decode_noalloc(
        q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(), op.bits.data_ptr(), k.data_ptr(), v.data_ptr(),
        out["features"].data_ptr(), out["valid"].data_ptr(), out["raw"].data_ptr(), out["ids"].data_ptr(),
        out["count"].data_ptr(), out["out"].data_ptr(), out["err"].data_ptr(), groups, history,
        k.shape[1] - history, op.capacity, op.row_words, k.stride(0), v.stride(0), op.capacity,
        torch.cuda.current_stream().cuda_stream)
    return rc, out


def _compare(op, q, k, v):
    ref = op(q, k, v)
    torch.cuda.synchronize()
    rc, got = _noalloc(op, q, k, v)
    torch.cuda.synchronize()
    assert rc == 0, rc
    assert int(got["err"].item()) == 0
    count = op.count.cpu().numpy()
    assert np.array_equal(count, got["count"].cpu().numpy())
    assert torch.equal(op.features, got["features"]) and torch.equal(op.valid, got["valid"])
    assert torch.equal(op.raw, got["raw"])
    ids, gids = op.ids.cpu().numpy(), got["ids"].cpu().numpy()
    for g in range(8):
        assert np.array_equal(ids[g, :count[g]], gids[g, :count[g]]), g
    assert torch.equal(ref.view(torch.int16), got["out"].view(torch.int16))
    log(f"  noalloc == decode: unique={count.tolist()}")


def test_noalloc_matches_decode_twice():
    big = cases.native_case(8192, 96, "random")
    small = cases.native_case(1025, 3, "random")
    for case in (big, small):
        log(f"case H={case['H']} T={case['T']}")
        op, q, k, v = operator(case)
        assert op.lib.query("prismkv_scratch_bytes") == 1 << 20
        _compare(op, q, k, v)


def test_noalloc_rejects_too_many_groups():
    case = cases.native_case(1025, 3, "random")
    op, q, k, v = operator(case)
    rc, _ = _noalloc(op, q, k, v, groups=14)  # the workspace of 14 groups exceeds the 1 MiB array
    assert rc == -1
    # a history the decode cannot take is refused by the same host checks as
    # prismkv_decode's, before the array is cleared: nothing is enqueued, and
    # the next call still matches prismkv_decode
    for bad in (0, op.capacity + 1):
        rc, got = _noalloc(op, q, k, v, history=bad)
        torch.cuda.synchronize()
        assert rc == -1, bad
        assert int(got["count"].abs().sum()) == 0 and int(got["err"].item()) == 0
    _compare(op, q, k, v)
