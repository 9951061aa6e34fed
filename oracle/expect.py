"""Expected route / union / attention results for a case -- TEST INFRASTRUCTURE ONLY.

`expected(case)` runs the oracle restatement of the reference decode step for
every KV group of a case (src/prismkv/core.py:106-183 via the C oracle) and
`compare(...)` checks device outputs against it:

* bucket features (rank order), raw, unique IDs and count must be identical
  -- when a group's rank margin (smallest relative gap between neighbouring
  scores in the top-17) is at least `margin_floor`; exact ties are broken by
  bucket id on both sides and need no margin;
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
                           ids=ids, margin=margin, ties=ties, meta=meta))
    return groups


def expected_attention(case, groups):
    k = bf16_to_f32(case["k"]) if case["k"].dtype == np.uint16 else case["k"]
    v = bf16_to_f32(case["v"]) if case["v"].dtype == np.uint16 else case["v"]
    q = bf16_to_f32(case["q"]) if case["q"].dtype == np.uint16 else case["q"]
    return np.stack([attend(q[g], k[g], v[g], groups[g]["ids"], case["H"]) for g in range(len(groups))])


def compare_route(groups, features, valid, raw, ids, count, margin_floor=MARGIN_FLOOR):
    """Returns (n_checked, n_skipped_for_margin); raises AssertionError on a mismatch."""
    checked = skipped = 0
    for g, e in enumerate(groups):
        if e["margin"] < margin_floor:
            skipped += 1
            continue
        n = len(e["order"])
        assert np.array_equal(features[g][:n], e["order"]), ("feature mismatch", g, features[g][:n], e["order"])
        assert np.array_equal(features[g][n:], np.zeros(TOPK - n, np.int64)), ("padding ids", g)
        assert np.array_equal(valid[g], e["valid"]), ("valid mismatch", g)
        assert int(raw[g]) == e["raw"], ("raw mismatch", g, int(raw[g]), e["raw"])
        assert int(count[g]) == len(e["ids"]), ("count mismatch", g, int(count[g]), len(e["ids"]))
        assert np.array_equal(ids[g][:len(e["ids"])].astype(np.int64), e["ids"]), ("ID mismatch", g)
        checked += 1
    return checked, skipped


def attention_errors(actual_bf16_bits, expected_f64):
    """relL2 / max-abs of the device output vs the fp64 oracle and vs the
    oracle rounded to bf16 (the reference casts to q.dtype, core.py:183)."""
    a = bf16_to_f32(actual_bf16_bits).astype(np.float64)
    ref_bf16 = bf16_to_f32(f32_to_bf16(expected_f64.astype(np.float32))).astype(np.float64)
    return dict(rel_l2=rel_l2(a, expected_f64), max_abs=float(np.abs(a - expected_f64).max()),
                rel_l2_vs_bf16=rel_l2(a, ref_bf16))
