"""Expected route / union / attention results for a case -- TEST INFRASTRUCTURE ONLY.

`expected(case)` runs the oracle restatement of the reference decode step for
every KV group of a case (src/prismkv/core.py:106-183 via the C oracle) and
`compare(...)` checks device outputs against it:

* bucket features (rank order), raw, unique IDs and count must be identical
  to the oracle's.  Where the device order differs from the oracle's, every
  differing rank must hold a bucket whose oracle score lies within the fp32
  rounding bound (`margin_floor`, relative) of the oracle's score at that
  rank -- a near-tie decided by summation order -- and raw / IDs / count must
  then equal the oracle's union of exactly the buckets the device chose.
  Exact ties are broken by bucket id on both sides and need no tolerance;
* the attention output must be within relative L2 `tol` (2e-3) of the fp64
  oracle, as the reference's bf16 output is (reviewer_guide/validation.md:19-22).
"""
from __future__ import annotations

import numpy as np

from . import attend, bf16_to_f32, bucket_scores, rel_l2, select_buckets, f32_to_bf16

TOPK = 16
MARGIN_FLOOR = 1e-5
UNDERFLOW = 1e-30
AV_TOL = 2e-3


def expected(case, unique_cap=None):
    q = bf16_to_f32(case["q"]) if case["q"].dtype == np.uint16 else case["q"]
    groups = []
    for g, idx in enumerate(case["indices"]):
        score, order, margin, ties = bucket_scores(q[g], idx.counts, idx.mean, idx.variance, topk=TOPK)
        live = np.sort(score[idx.counts > 0])[::-1]
        if len(live) and live[min(len(live), TOPK + 1) - 1] < UNDERFLOW:
            margin = 0.0   # ranks decided below fp32 resolution: order is implementation-defined
        ids, meta = select_buckets(order, idx.lists, case["H"], unique_cap)
        feats = np.zeros(TOPK, np.int64)
        valid = np.zeros(TOPK, np.float32)
        feats[:len(order)] = order
        valid[:len(order)] = 1
        groups.append(dict(order=order, features=feats, valid=valid, raw=int(idx.counts[order].sum()),
                           ids=ids, margin=margin, ties=ties, meta=meta, score=score, counts=idx.counts,
                           lists=idx.lists, H=case["H"]))
    return groups


def expected_attention(case, groups):
    k = bf16_to_f32(case["k"]) if case["k"].dtype == np.uint16 else case["k"]
    v = bf16_to_f32(case["v"]) if case["v"].dtype == np.uint16 else case["v"]
    q = bf16_to_f32(case["q"]) if case["q"].dtype == np.uint16 else case["q"]
    return np.stack([attend(q[g], k[g], v[g], groups[g]["ids"], case["H"]) for g in range(len(groups))])


def compare_route(groups, features, valid, raw, ids, count, margin_floor=MARGIN_FLOOR, allow_near=False,
                  swaps=None):
    """Returns (n_identical, n_near_tie); raises AssertionError on a mismatch.

    n_identical groups match the oracle's order exactly.  With allow_near
    (only for cases built to hold ties decided by fp32 summation order), a
    group may instead choose a different order among buckets whose oracle
    scores agree to within `margin_floor` (relative) or both lie below
    UNDERFLOW; it then counts as a near tie, its raw / IDs / count must equal
    the oracle's union of the device's choice, and every swapped rank is
    appended to `swaps` (a list, if given) as (group, rank, oracle bucket,
    device bucket, relative score gap).  Without allow_near any difference
    from the oracle's order fails."""
    identical = near = 0
    for g, e in enumerate(groups):
        n = len(e["order"])
        got = np.asarray(features[g][:n], np.int64)
        assert np.array_equal(features[g][n:], np.zeros(TOPK - n, np.int64)), ("padding ids", g)
        assert np.array_equal(valid[g], e["valid"]), ("valid mismatch", g)
        if np.array_equal(got, e["order"]):
            want_ids, want_raw = e["ids"], e["raw"]
            identical += 1
        else:
            assert allow_near, ("feature order differs from the oracle's", g, got.tolist(), e["order"].tolist(),
                                "margin", e["margin"])
            assert len(np.unique(got)) == n and got.min() >= 0 and got.max() < len(e["counts"]), ("bad ids", g, got)
            assert np.all(e["counts"][got] > 0), ("dead bucket selected", g, got)
            sc = e["score"]
            want_sc, got_sc = sc[e["order"]], sc[got]
            tol = margin_floor * np.abs(want_sc) + UNDERFLOW
            bad = np.abs(got_sc - want_sc) > tol
            assert not bad.any(), ("feature mismatch beyond near-tie tolerance", g, got, e["order"],
                                   got_sc[bad], want_sc[bad])
            if swaps is not None:
                for r in np.flatnonzero(got != e["order"]):
                    gap = abs(float(got_sc[r]) - float(want_sc[r])) / max(abs(float(want_sc[r])), UNDERFLOW)
                    swaps.append((g, int(r), int(e["order"][r]), int(got[r]), gap))
            want_ids, _ = select_buckets(got, e["lists"], e["H"])
            want_raw = int(e["counts"][got].sum())
            near += 1
        assert int(raw[g]) == want_raw, ("raw mismatch", g, int(raw[g]), want_raw)
        assert int(count[g]) == len(want_ids), ("count mismatch", g, int(count[g]), len(want_ids))
        assert np.array_equal(ids[g][:len(want_ids)].astype(np.int64), want_ids), ("ID mismatch", g)
    return identical, near


def attention_errors(actual_bf16_bits, expected_f64):
    """relL2 / max-abs of the device output vs the fp64 oracle and vs the
    oracle rounded to bf16 (the reference casts to q.dtype, core.py:183)."""
    a = bf16_to_f32(actual_bf16_bits).astype(np.float64)
    ref_bf16 = bf16_to_f32(f32_to_bf16(expected_f64.astype(np.float32))).astype(np.float64)
    return dict(rel_l2=rel_l2(a, expected_f64), max_abs=float(np.abs(a - expected_f64).max()),
                rel_l2_vs_bf16=rel_l2(a, ref_bf16))


def encode_error_bound(x, W, b):
    """A-priori bound on |device fp32 encode - oracle encode| of relu(x W^T + b)
    (src/prismkv/core.py:47-48) over all entries: a 128-term fp32 dot product
    and the bias add carry at most (d + 2) u sum_i |x_i W_fi| + u |b_f| of
    rounding (u = 2^-24, any summation order); the oracle accumulates in
    float64 (negligible)."""
    x = np.abs(np.asarray(x, np.float64))
    W = np.abs(np.asarray(W, np.float64))
    d = x.shape[1]
    u = 2.0 ** -24
    return float(((d + 2) * u * (x @ W.T) + u * np.abs(np.asarray(b, np.float64))[None, :]).max())


def membership_flat(lists, H):
    """Sorted flat indices token * F + feature of per-feature token lists."""
    F = len(lists)
    parts = [np.asarray(l, np.int64) * F + f for f, l in enumerate(lists) if len(l)]
    flat = np.concatenate(parts) if parts else np.zeros(0, np.int64)
    assert flat.size == 0 or (flat.min() >= 0 and flat.max() < H * F)
    return np.sort(flat)


def check_memberships(ref_lists, dev_lists, act_ref, count, bound, tag=""):
    """BatchTopK memberships of the device vs the oracle (core.py:13-26).

    Identical lists pass.  Otherwise every (token, feature) membership that is
    on one side only must have an oracle activation within 2 * `bound` of the
    oracle's threshold tau (the count-th largest activation): the device's
    activation and its tau each lie within `bound` of the oracle's, so only
    such entries can change sides.  Returns the number of differing
    memberships (logged by the caller)."""
    H, F = act_ref.shape
    a = membership_flat(ref_lists, H)
    b = membership_flat(dev_lists, H)
    diff = np.setxor1d(a, b, assume_unique=True)
    if diff.size == 0:
        return 0
    vals = np.asarray(act_ref, np.float32).reshape(-1)
    count = min(int(count), vals.size)
    tau = float(np.partition(vals, vals.size - count)[vals.size - count])
    gap = np.abs(vals[diff].astype(np.float64) - tau)
    worst = int(np.argmax(gap))
    assert gap[worst] <= 2 * bound, ("membership differs away from tau", tag, int(diff[worst] // F),
                                     int(diff[worst] % F), float(gap[worst]), 2 * bound)
    return int(diff.size)
