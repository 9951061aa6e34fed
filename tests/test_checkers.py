"""CPU checks of the parity checkers themselves: mistakes planted in the
oracle's own outputs must be caught.

The GPU tests compare device outputs against `oracle.expect.compare_route`
and `oracle.expect.check_memberships`; these tests feed those checkers the
oracle's results with one deliberate change each (a swapped rank, a dropped
id, a membership moved away from the threshold) and require a failure, and
require the legitimate near-tie cases to pass only where they are allowed.
"""
import numpy as np
import pytest

import oracle
from oracle import cases, expect


@pytest.fixture(scope="module")
def routed(oracle_lib):
    case = cases.native_case(1025, 3, "random")
    groups = expect.expected(case)
    G, H = 8, case["H"]
    features = np.stack([g["features"] for g in groups])
    valid = np.stack([g["valid"] for g in groups])
    raw = np.array([g["raw"] for g in groups], np.int32)
    ids = np.zeros((G, H), np.int32)
    count = np.zeros(G, np.int32)
    for i, g in enumerate(groups):
        ids[i, :len(g["ids"])] = g["ids"]
        count[i] = len(g["ids"])
    return groups, features, valid, raw, ids, count


def _copy(t):
    return tuple(np.array(x, copy=True) for x in t)


def test_oracle_outputs_pass(routed):
    groups, *out = routed
    assert expect.compare_route(groups, *_copy(out)) == (8, 0)


def test_swapped_ranks_fail(routed):
    groups, *out = routed
    features, valid, raw, ids, count = _copy(out)
    features[2, [4, 5]] = features[2, [5, 4]]  # distinct scores: a real ranking error
    with pytest.raises(AssertionError):
        expect.compare_route(groups, features, valid, raw, ids, count)
    with pytest.raises(AssertionError):  # beyond the near-tie tolerance too
        expect.compare_route(groups, features, valid, raw, ids, count, allow_near=True)


def test_wrong_ids_raw_count_fail(routed):
    groups, *out = routed
    for what in ("ids", "raw", "count", "valid"):
        features, valid, raw, ids, count = _copy(out)
        if what == "ids":
            ids[1, 3] += 1
        elif what == "raw":
            raw[6] += 1
        elif what == "count":
            count[0] -= 1
        else:
            valid[3, 0] = 0
        with pytest.raises(AssertionError):
            expect.compare_route(groups, features, valid, raw, ids, count)


def test_near_tie_swap_only_when_allowed(routed):
    groups, *out = routed
    features, valid, raw, ids, count = _copy(out)
    g = dict(groups[5])
    score = g["score"].copy()
    a, b = int(g["order"][7]), int(g["order"][8])
    score[b] = score[a] * (1 - 1e-7)  # make ranks 7 and 8 a near tie in the oracle's scores
    g["score"] = score
    gs = list(groups)
    gs[5] = g
    features[5, [7, 8]] = features[5, [8, 7]]
    # the union of the same buckets: ids / raw / count are unchanged
    with pytest.raises(AssertionError):
        expect.compare_route(gs, features, valid, raw, ids, count)
    swaps = []
    assert expect.compare_route(gs, features, valid, raw, ids, count, allow_near=True, swaps=swaps) == (7, 1)
    assert [(s[0], s[1]) for s in swaps] == [(5, 7), (5, 8)] and max(s[4] for s in swaps) < 1e-6


def _memberships(act, count):
    H, F = act.shape
    flat = oracle.positive_global_topk(act, count)
    lists = [[] for _ in range(F)]
    for x in flat:
        lists[int(x % F)].append(int(x // F))
    return [np.array(sorted(l), np.int64) for l in lists]


def test_check_memberships(oracle_lib):
    rng = np.random.default_rng(3)
    H, F, count = 40, 3000, 320
    act = np.maximum(rng.standard_normal((H, F)).astype(np.float32), 0)
    ref = _memberships(act, count)
    assert expect.check_memberships(ref, [l.copy() for l in ref], act, count, 1e-6) == 0
    vals = act.reshape(-1)
    tau = float(np.partition(vals, vals.size - count)[vals.size - count])
    # a membership traded across the threshold by rounding: allowed
    below = int(np.argmax(np.where(vals < tau, vals, -1)))  # the largest value below tau
    at = int(np.argmin(np.where(vals >= tau, vals, np.inf)))  # the smallest selected value
    near = [l.copy() for l in ref]
    near[at % F] = near[at % F][near[at % F] != at // F]
    near[below % F] = np.sort(np.append(near[below % F], below // F))
    gap = max(abs(vals[below] - tau), abs(vals[at] - tau))
    assert expect.check_memberships(ref, near, act, count, gap) == 2
    # a membership far from the threshold: caught
    far = [l.copy() for l in ref]
    small = int(np.argmin(np.where(vals > 0, vals, np.inf)))
    far[small % F] = np.sort(np.append(far[small % F], small // F))
    with pytest.raises(AssertionError):
        expect.check_memberships(ref, far, act, count, 1e-4)


def test_encode_error_bound_covers_fp32(oracle_lib):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((64, 128)).astype(np.float32)
    W = (rng.standard_normal((300, 128)) / np.sqrt(128)).astype(np.float32)
    b = rng.standard_normal(300).astype(np.float32) * 0.1
    exact = np.maximum(x.astype(np.float64) @ W.T.astype(np.float64) + b, 0)
    fp32 = np.maximum((x @ W.T).astype(np.float32) + b, 0)  # any fp32 summation order
    bound = expect.encode_error_bound(x, W, b)
    assert np.abs(fp32 - exact).max() <= bound
    assert np.abs(oracle.sae_dense(x, W, b) - exact).max() <= bound
