"""Pins the C oracle to the reference's own known-answer tests.

Each test restates one case of tests/test_core.py (the reference suite) with
the literal inputs and expected values found there, run through the oracle
instead of src/prismkv/core.py.
"""
import numpy as np
import pytest

import oracle
from oracle import cases


def test_global_budget_variable_cardinality_and_zero(oracle_lib):
    # tests/test_core.py:12-17
    a = np.array([[10., 9., 8., 7.], [1., .9, .8, .7]], np.float32)
    ids = oracle.positive_global_topk(a, 4)
    assert (ids // 4).tolist() == [0, 0, 0, 0]
    assert len(oracle.positive_global_topk(np.zeros_like(a), 4)) == 0
    assert oracle.positive_global_topk(np.ones((2, 4), np.float32), 3).tolist() == [0, 1, 2]


def test_moments_of_original_keys_and_empty_bucket(oracle_lib):
    # tests/test_core.py:26-33
    k = np.array([[2., 4.], [4., 8.], [9., 0.]], np.float32)
    counts, mean, var = oracle.summarize(k, [np.array([0, 1]), np.array([2]), np.array([], np.int64)])
    np.testing.assert_allclose(mean[0], [3., 6.])
    np.testing.assert_allclose(var[0], [1., 4.])
    assert counts.tolist() == [2, 1, 0]
    score, _, _, _ = oracle.bucket_scores(np.ones((1, 2), np.float32), counts, mean, var)
    assert score[-1] == 0


def test_gqa_normalize_before_aggregation(oracle_lib):
    # tests/test_core.py:35-42
    k = np.array([[10., 0.], [0., 2.], [-3., -1.]], np.float32)
    counts, mean, var = oracle.summarize(k, [np.array([0]), np.array([1]), np.array([2])])
    q = np.array([[1., 0.], [0., 1.]], np.float32)
    score, _, _, _ = oracle.bucket_scores(q, counts, mean, var, topk=3, terms=("mean",))
    logits = q.astype(np.float64) @ k.T.astype(np.float64) / np.sqrt(2)
    sm = np.exp(logits - logits.max(-1, keepdims=True))
    wanted = (sm / sm.sum(-1, keepdims=True)).mean(0)
    np.testing.assert_allclose(score, wanted, rtol=1e-12)
    avg = logits.mean(0)
    other = np.exp(avg - avg.max()) / np.exp(avg - avg.max()).sum()
    assert np.abs(wanted - other).max() > .01


def test_overlap_unique_budget_skips_overflow(oracle_lib):
    # tests/test_core.py:44-53
    keys = np.zeros((10, 2), np.float32)
    lists = [np.array([0, 1, 2, 3]), np.array([2, 3]), np.array([4])]
    counts, mean, var = oracle.summarize(keys, lists)
    q = np.ones((1, 2), np.float32)
    _, order, _, _ = oracle.bucket_scores(q, counts, mean, var, topk=3, terms=("count",))
    ids, meta = oracle.select_buckets(order, lists, 10, unique_cap=.3)
    assert ids.tolist() == [2, 3, 4]
    assert meta["features"] == [1, 2]
    assert meta["raw"] == 3
    _, order, _, _ = oracle.bucket_scores(q, counts, mean, var, topk=2, terms=("count",))
    full_ids, meta = oracle.select_buckets(order, lists, 10)
    assert full_ids.tolist() == [0, 1, 2, 3]
    assert meta["raw"] == 6


def test_full_and_selected_original_attention_with_dense_tail(oracle_lib):
    # tests/test_core.py:55-63 (random inputs; expected value by direct softmax)
    rng = np.random.default_rng(37)
    k, v, q = (rng.standard_normal((9, 4)).astype(np.float32), rng.standard_normal((9, 4)).astype(np.float32),
               rng.standard_normal((3, 4)).astype(np.float32))

    def direct(rows):
        lg = q.astype(np.float64) @ k[rows].T.astype(np.float64) / 2
        p = np.exp(lg - lg.max(-1, keepdims=True))
        return (p / p.sum(-1, keepdims=True)) @ v[rows].astype(np.float64)

    np.testing.assert_allclose(oracle.attend(q, k, v, np.arange(6), 6), direct(np.arange(9)), rtol=1e-12)
    chosen = np.array([1, 3, 6, 7, 8])
    np.testing.assert_allclose(oracle.attend(q, k, v, np.array([1, 3]), 6), direct(chosen), rtol=1e-12)
    with pytest.raises(ValueError):
        oracle.attend(q, k, v, np.array([1, 1]), 6)


def test_empty_index_and_zero_budget(oracle_lib):
    # tests/test_core.py:65-72
    rng = np.random.default_rng(1)
    k = rng.standard_normal((5, 2)).astype(np.float32)
    counts, mean, var = oracle.summarize(k, [np.array([], np.int64)])
    _, order, _, _ = oracle.bucket_scores(np.ones((1, 2), np.float32), counts, mean, var)
    ids, _ = oracle.select_buckets(order, [np.array([], np.int64)], 5)
    assert len(ids) == 0
    lists = [np.arange(5)]
    counts, mean, var = oracle.summarize(k, lists)
    _, order, _, _ = oracle.bucket_scores(np.ones((1, 2), np.float32), counts, mean, var)
    ids, _ = oracle.select_buckets(order, lists, 5, unique_cap=0)
    assert len(ids) == 0


def test_incremental_moments_preserve_old_memberships(oracle_lib):
    # tests/test_core.py:74-86 (SharedSAE(4, 12, 2, 3): d=4, F=12, key_mean=2)
    rng = np.random.default_rng(37)
    k = rng.standard_normal((17, 4)).astype(np.float32)
    new = (rng.standard_normal((7, 4)) + 4).astype(np.float32)
    W = rng.uniform(-.5, .5, (12, 4)).astype(np.float32)
    b = np.zeros(12, np.float32)
    index = oracle.build_index(k, W, b, 1.0, key_mean=2)
    before = [x.copy() for x in index.lists]
    merged = oracle.append_index(index, new, W, b, 1.0, key_mean=2)
    counts, mean, var = oracle.summarize(np.concatenate((k, new)), merged.lists)
    np.testing.assert_allclose(merged.mean, mean, atol=1e-6, rtol=1e-5)
    np.testing.assert_allclose(merged.variance, var, atol=1e-5, rtol=1e-5)
    assert np.array_equal(merged.counts, counts)
    for old, ids in zip(before, merged.lists):
        assert np.array_equal(ids[:len(old)], old)
    assert merged.memberships - index.memberships == 7 * 2
    assert np.array_equal(merged.center, index.center)


def test_native_witness_membership_counts(oracle_lib):
    # reviewer_guide/native8b_validation.json: memberships per group for the
    # six cases of examples/check_native8b.py:80
    for H, tail, kind in cases.NATIVE_CASES:
        lists = cases.native_lists(H, kind, 0)
        assert sum(len(x) for x in lists) == cases.NATIVE_MEMBERSHIPS[(H, kind)]
        for l in lists:
            assert np.all(np.diff(l) > 0)
