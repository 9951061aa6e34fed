"""Pins the C oracle where the reference's own tests leave it open: brute
force on small inputs, closed forms, invariants and library routines
(scipy/numpy), chosen so a dropped term, wrong sign/index or transposed
operand in the oracle fails at least one of them."""
import numpy as np
import pytest
from scipy.special import softmax

import oracle
from oracle import cases


def brute_topk(a, count):
    flat = a.reshape(-1)
    count = min(count, flat.size)
    if count == 0:
        return np.zeros(0, np.int64)
    thr = np.sort(flat)[::-1][count - 1]
    strict = np.nonzero((flat > thr) & (flat > 0))[0]
    if thr > 0:
        ties = np.nonzero(flat == thr)[0][:count - len(strict)]
        return np.concatenate((strict, ties))
    return strict


@pytest.mark.parametrize("seed", range(6))
def test_batch_topk_matches_brute_force(oracle_lib, seed):
    rng = np.random.default_rng(seed)
    a = np.maximum(rng.standard_normal((37, 53)), 0).astype(np.float32)
    # plant ties at several levels, including at the threshold
    a.flat[rng.choice(a.size, 40, replace=False)] = np.float32(0.75)
    a.flat[rng.choice(a.size, 15, replace=False)] = np.float32(1.5)
    for count in (0, 1, 7, 64, 200, 900, a.size, a.size + 5):
        got = oracle.positive_global_topk(a, count)
        assert np.array_equal(got, brute_topk(a, count)), count


def test_batch_topk_negative_and_zero_threshold(oracle_lib):
    a = np.array([[3., -1., 0.], [2., -5., 0.]], np.float32)
    assert oracle.positive_global_topk(a, 4).tolist() == [0, 3]   # threshold 0: positives only
    assert oracle.positive_global_topk(-np.abs(a) - 1, 2).tolist() == []


def test_topk_margin(oracle_lib):
    a = np.array([[5., 4., 3., 1.]], np.float32)
    assert oracle.topk_margin(a, 2) == pytest.approx(0.25)   # threshold 4, neighbours 5 and 3


def test_union_is_set_union_and_bitmap_round_trip(oracle_lib):
    rng = np.random.default_rng(3)
    H, F = 1000, 40
    lists = [np.unique(rng.integers(0, H, rng.integers(0, 60))) for _ in range(F)]
    bits = oracle.build_bits(lists, (H + 31) // 32 + 5)
    for f in range(F):   # bits -> members
        row = np.unpackbits(bits[f].view(np.uint8), bitorder="little")
        assert np.array_equal(np.nonzero(row)[0], lists[f])
    feats = rng.choice(F, 16, replace=False)
    valid = (rng.random(16) > .3).astype(np.float32)
    got = oracle.union_bits(bits, H, feats, valid)
    want = sorted(set().union(*[set(lists[f].tolist()) for f, v in zip(feats, valid) if v > 0]))
    assert got.tolist() == want


def test_select_buckets_properties(oracle_lib):
    rng = np.random.default_rng(4)
    H = 500
    lists = [np.unique(rng.integers(0, H, rng.integers(1, 80))) for _ in range(30)]
    order = rng.permutation(30)[:16]
    full, meta = oracle.select_buckets(order, lists, H)
    assert full.tolist() == sorted(set().union(*[set(lists[b].tolist()) for b in order]))
    assert meta["raw"] == sum(len(lists[b]) for b in order)
    assert meta["features"] == order.tolist()
    same, _ = oracle.select_buckets(order, lists, H, unique_cap=1.0)
    assert np.array_equal(same, full)
    for cap in (.02, .05, .1, .2):
        ids, meta = oracle.select_buckets(order, lists, H, unique_cap=cap)
        assert len(ids) <= np.floor(H * cap) and set(ids.tolist()) <= set(full.tolist())
        assert set(ids.tolist()) == set().union(*[set(lists[b].tolist()) for b in meta["features"]])
    with pytest.raises(ValueError):
        oracle.select_buckets(order, lists, H, unique_cap=1.5)


def test_count_only_route_is_count_share(oracle_lib):
    # softmax over log(n) is n / sum(n): closed form, independent of q
    rng = np.random.default_rng(5)
    counts = rng.integers(0, 50, 200)
    counts[::7] = 0
    mean = rng.standard_normal((200, 8)).astype(np.float32)
    var = rng.random((200, 8)).astype(np.float32)
    q = rng.standard_normal((4, 8)).astype(np.float32)
    score, order, _, _ = oracle.bucket_scores(q, counts, mean, var, topk=16, terms=("count",))
    np.testing.assert_allclose(score, counts / counts.sum(), rtol=1e-12)
    want = np.lexsort((np.arange(200), -counts))
    want = [b for b in want if counts[b] > 0][:16]
    assert order.tolist() == want


def test_mean_and_variance_terms_against_scipy(oracle_lib):
    rng = np.random.default_rng(6)
    F, d = 300, 16
    counts = rng.integers(1, 30, F)
    mean = rng.standard_normal((F, d)).astype(np.float32)
    var = rng.random((F, d)).astype(np.float32)
    q = rng.standard_normal((3, d)).astype(np.float32)
    q64, m64, v64 = q.astype(np.float64), mean.astype(np.float64), var.astype(np.float64)
    for terms, logits in [(("mean",), q64 @ m64.T / np.sqrt(d)),
                          (("variance",), (q64 ** 2) @ v64.T / (2 * d)),
                          (("count", "mean", "variance"),
                           np.log(counts)[None] + q64 @ m64.T / np.sqrt(d) + (q64 ** 2) @ v64.T / (2 * d))]:
        score, order, margin, _ = oracle.bucket_scores(q, counts, mean, var, topk=16, terms=terms)
        want = softmax(logits, axis=-1).mean(0)
        np.testing.assert_allclose(score, want, rtol=1e-10, atol=1e-15)
        assert order.tolist() == np.argsort(-want, kind="stable")[:16].tolist()
        assert margin > 0


def test_norm_top_agrees_with_bucket_scores(oracle_lib):
    # the native route (prescaled products + log count) ranks like core.bucket_scores
    rng = np.random.default_rng(7)
    F, d = 3000, 128
    counts = rng.integers(0, 40, F)
    mean = rng.standard_normal((F, d)).astype(np.float32) * .3
    var = rng.random((F, d)).astype(np.float32)
    q = rng.standard_normal((4, d)).astype(np.float32)
    _, order, margin, _ = oracle.bucket_scores(q, counts, mean, var)
    a = np.concatenate((q, q * q), -1).astype(np.float64)
    matrix = np.concatenate((mean.T / np.sqrt(128), var.T / 256)).astype(np.float64)
    prod = (a @ matrix).astype(np.float32)
    ln = np.log(np.maximum(counts, 1)).astype(np.float32)
    ids, vals, raw, margin2, _ = oracle.norm_top(prod, ln, counts.astype(np.int32))
    assert margin > 1e-4 and margin2 > 1e-4
    assert ids.tolist() == order.tolist() and vals.tolist() == [1.0] * 16
    assert raw == counts[order].sum()


def test_norm_top_padding_and_ties(oracle_lib):
    ct = np.zeros(3000, np.int32)
    ct[[5, 9, 2000]] = 3
    prod = np.zeros((4, 3000), np.float32)
    ids, vals, raw, _, ties = oracle.norm_top(prod, np.log(np.maximum(ct, 1)).astype(np.float32), ct)
    assert ids.tolist() == [5, 9, 2000] + [0] * 13
    assert vals.tolist() == [1.0] * 3 + [0.0] * 13
    assert raw == 9 and ties == 2


def test_attend_special_cases(oracle_lib):
    rng = np.random.default_rng(8)
    k = rng.standard_normal((10, 6)).astype(np.float32)
    v = rng.standard_normal((10, 6)).astype(np.float32)
    q = rng.standard_normal((2, 6)).astype(np.float32)
    # one row -> that V row
    np.testing.assert_allclose(oracle.attend(q, k, v, np.array([3]), 10), np.repeat(v[3:4], 2, 0), rtol=1e-12)
    # identical keys -> plain average of V rows
    kk = np.repeat(k[:1], 10, 0)
    np.testing.assert_allclose(oracle.attend(q, kk, v, np.array([0, 4, 7]), 8),
                               np.repeat(v[[0, 4, 7, 8, 9]].astype(np.float64).mean(0, keepdims=True), 2, 0), rtol=1e-12)
    # general case vs scipy softmax, row order irrelevant
    rows = np.array([2, 5, 6, 8, 9])
    want = softmax(q.astype(np.float64) @ k[rows].T.astype(np.float64) / np.sqrt(6), axis=-1) @ v[rows]
    np.testing.assert_allclose(oracle.attend(q, k, v, np.array([6, 2, 5]), 8), want, rtol=1e-12)
    # nothing to read -> zeros
    assert np.all(oracle.attend(q, k, v, np.zeros(0, np.int64), 10) == 0)
    with pytest.raises(ValueError):
        oracle.attend(q, k, v, np.array([8]), 8)


def test_merge_moments_equals_recompute(oracle_lib):
    rng = np.random.default_rng(9)
    keys = (rng.standard_normal((300, 5)) * 2 + 1).astype(np.float32)
    la = [np.unique(rng.integers(0, 200, rng.integers(0, 30))) for _ in range(20)]
    lb = [np.unique(rng.integers(200, 300, rng.integers(0, 10))) for _ in range(20)]
    ca, ma, va = oracle.summarize(keys, la)
    cb, mb, vb = oracle.summarize(keys, lb)
    co, mo, vo = oracle.merge_moments(ca, ma, va, cb, mb, vb)
    cw, mw, vw = oracle.summarize(keys, [np.concatenate((a, b)) for a, b in zip(la, lb)])
    assert np.array_equal(co, cw)
    np.testing.assert_allclose(mo, mw, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(vo, vw, rtol=1e-5, atol=1e-5)


def test_sae_dense_and_pack(oracle_lib):
    rng = np.random.default_rng(10)
    x = rng.standard_normal((9, 16)).astype(np.float32)
    W = rng.standard_normal((30, 16)).astype(np.float32)
    b = rng.standard_normal(30).astype(np.float32)
    want = np.maximum(x.astype(np.float64) @ W.T.astype(np.float64) + b, 0)
    np.testing.assert_allclose(oracle.sae_dense(x, W, b), want, rtol=1e-6, atol=1e-6)
    qb = oracle.f32_to_bf16(rng.standard_normal((32, 128)).astype(np.float32))
    a = oracle.pack(qb)
    qf = oracle.bf16_to_f32(qb)
    assert np.array_equal(a[:, :128], qf) and np.array_equal(a[:, 128:], qf * qf)


def test_bf16_round_trip_and_rne():
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.4e38, np.inf], np.float32)
    # 1 + 2^-8 is a tie between 1 and 1+2^-7: rounds to even (1.0)
    assert oracle.bf16_to_f32(oracle.f32_to_bf16(x)).tolist()[:4] == [1.0, 1.0, 1.015625, -2.5]


def test_native_witness_unique_counts(oracle_lib):
    # reviewer_guide/native8b_validation.json: for "ties", "few" and "empty" the
    # unique counts do not depend on the random K/Q (16, 65, 0 in every group)
    for H, tail, kind, want in [(32, 1, "ties", 16), (65, 7, "few", 65), (257, 129, "empty", 0)]:
        from oracle import expect
        case = cases.native_case(H, tail, kind)
        for e in expect.expected(case):
            assert len(e["ids"]) == want


# ---------------------------------------------------------------- q_activation router

def _unit_sae(F=3000, d=128):
    """W with row f = e_(f mod d) for f < d, zero rows beyond: a[h][f] = relu(x[h][f]) for f < d, else relu(b)."""
    W = np.zeros((F, d), np.float32)
    W[np.arange(d), np.arange(d)] = 1.0
    return W, np.zeros(F, np.float32)


def test_qact_scores_properties():
    rng = np.random.default_rng(11)
    W = (rng.standard_normal((3000, 128)) / np.sqrt(128)).astype(np.float32)
    b = (rng.standard_normal(3000) * 0.1).astype(np.float32)
    q = rng.standard_normal((4, 128)).astype(np.float32)
    counts = rng.integers(0, 3, 3000).astype(np.int64)
    score, order, margin = oracle.qact_scores(q, W, b, 1.5, counts)
    # every head's weights sum to 1/4 (core.py:137-138), so the scores sum to 1
    assert abs(float(score.astype(np.float64).sum()) - 1.0) < 1e-5
    # the order: exactly the live positive-score buckets, score descending then id ascending
    live = np.flatnonzero((score > 0) & (counts > 0))
    want = live[np.lexsort((live, -score[live].astype(np.float64)))]
    assert np.array_equal(order, want)
    # independent recomputation in float64 with argsort (a different route to the same numbers)
    x = q.astype(np.float64) / np.float32(1.5)
    a = np.maximum(x @ W.astype(np.float64).T + b, 0)
    ids = np.argsort(-a, axis=1, kind="stable")[:, :16]
    val = np.take_along_axis(a, ids, 1)
    val = val / np.maximum(val.sum(1, keepdims=True), 1e-20)
    ref = np.zeros(3000)
    np.add.at(ref, ids.ravel(), (val / 4).ravel())
    assert np.allclose(score, ref, rtol=1e-5, atol=1e-8)
    if margin > 1e-4:
        live2 = np.flatnonzero((ref > 0) & (counts > 0))
        assert np.array_equal(order, live2[np.argsort(-ref[live2], kind="stable")])


def test_qact_scores_ties_duplicates_and_empty():
    W, b = _unit_sae()
    counts = np.ones(3000, np.int64)
    # 20 equal activations in every head: the stable argsort keeps ids 0..15,
    # each weight (1/16)/4, and all four heads pick the same buckets: 4/64 each
    q = np.zeros((4, 128), np.float32)
    q[:, :20] = 2.0
    score, order, _ = oracle.qact_scores(q, W, b, 1.0, counts)
    assert np.array_equal(order, np.arange(16))
    assert np.allclose(score[:16], 1 / 16) and not score[16:].any()
    # fewer than 16 positive activations: the zero-valued picks weigh nothing
    q = np.zeros((4, 128), np.float32)
    q[0, 5], q[1, 7] = 3.0, 1.0
    counts[7] = 0  # an empty bucket keeps its score but leaves the order
    score, order, _ = oracle.qact_scores(q, W, b, 1.0, counts)
    assert np.array_equal(order, [5])
    assert np.isclose(score[5], 0.25) and np.isclose(score[7], 0.25)
    # no positive activation at all: the clamped sum gives zero scores, an empty order
    score, order, _ = oracle.qact_scores(np.zeros((4, 128), np.float32), W, b, 1.0, counts)
    assert len(order) == 0 and not score.any()
