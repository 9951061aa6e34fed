"""Pins the torch-CPU restatement (oracle/torch_cpu.py, the CPU baseline that
bench.py times) against the C oracle: the reference's known answers
(tests/test_core.py:12-17, :44-53, :55-63) and the replay shape of
examples/replay.py (8 groups, H=1024, T=32, global-budget index), where the
bucket order, union, kept buckets and raw must be identical, and scores and
attention agree to fp32 rounding."""
import numpy as np
import pytest
import torch

import oracle
from oracle import bf16_to_f32, cases, expect
from oracle import torch_cpu as tc


def test_batch_topk_known_answers(oracle_lib):
    # tests/test_core.py:12-17
    a = torch.tensor([[10., 9., 8., 7.], [1., .9, .8, .7]])
    assert (tc.batch_topk(a, 4) // 4).tolist() == [0, 0, 0, 0]
    assert tc.batch_topk(torch.zeros(2, 4), 4).numel() == 0
    assert tc.batch_topk(torch.ones(2, 4), 3).tolist() == [0, 1, 2]
    rng = np.random.default_rng(4)
    x = np.round(rng.standard_normal((50, 300)) * 4) / 4  # many ties at the threshold
    x = x.astype(np.float32)
    for budget in (0, 1, 17, 400, 15000, 20000):
        got = np.sort(tc.batch_topk(torch.from_numpy(x), budget).numpy())
        assert np.array_equal(got, np.sort(oracle.positive_global_topk(x, budget))), budget


def test_cap_walk_known_answer(oracle_lib):
    # tests/test_core.py:44-53
    lists = [torch.tensor([0, 1, 2, 3]), torch.tensor([2, 3]), torch.tensor([4])]
    counts = torch.tensor([4, 2, 1])
    zeros = torch.zeros(3, 2)
    _, order = tc.moment_route(torch.ones(1, 2), counts, zeros, zeros, topk=3)
    ids, kept, raw = tc.union_walk(order, lists, 10, unique_cap=.3)
    assert ids.tolist() == [2, 3, 4] and kept == [1, 2] and raw == 3
    ids, kept, raw = tc.union_walk(order[:2], lists, 10)
    assert ids.tolist() == [0, 1, 2, 3] and raw == 6


def test_tail_attention_known_answer():
    # tests/test_core.py:55-63: no old ids, the tail alone
    keys = torch.tensor([[1., 0.], [0., 1.]])
    values = torch.tensor([[2., 0.], [0., 4.]])
    out = tc.attend_rows(torch.tensor([[0., 0.]]), keys, values, torch.zeros(0, dtype=torch.long), 0)
    assert torch.allclose(out, torch.tensor([[1., 2.]]))


@pytest.mark.parametrize("cap", [None, 0.2])
def test_replay_shape_matches_oracle(oracle_lib, cap):
    case = cases.replay_case(seed=5, H=1024, T=32, bf16=False)
    H = case["H"]
    for g, idx in enumerate(case["indices"]):
        q = torch.from_numpy(case["q"][g])
        counts, mean, var = (torch.from_numpy(x) for x in (idx.counts, idx.mean, idx.variance))
        score, order = tc.moment_route(q, counts, mean, var)
        w_score, w_order, margin, _ = oracle.bucket_scores(case["q"][g], idx.counts, idx.mean, idx.variance)
        assert np.array_equal(order.numpy(), w_order), (g, margin)
        np.testing.assert_allclose(score.numpy(), w_score, rtol=1e-5, atol=1e-12)
        lists = [torch.from_numpy(np.asarray(l, np.int64)) for l in idx.lists]
        ids, kept, raw = tc.union_walk(order, lists, H, cap)
        w_ids, w_meta = oracle.select_buckets(w_order, idx.lists, H, cap)
        assert np.array_equal(ids.numpy(), w_ids) and kept == w_meta["features"] and raw == w_meta["raw"]
        out = tc.attend_rows(q, torch.from_numpy(case["k"][g]), torch.from_numpy(case["v"][g]), ids, H)
        want = oracle.attend(case["q"][g], case["k"][g], case["v"][g], w_ids, H)
        assert oracle.rel_l2(out.numpy().astype(np.float64), want) < 1e-5


def test_append_block_matches_oracle(oracle_lib):
    case = cases.update_case("random", H=512, N=256, T=8, seed=21)
    H, N = case["H"], case["N"]
    kf = bf16_to_f32(case["k"])
    for g in (0, 3):
        idx = case["indices"][g]
        W, b, s = case["W"][g], case["b"][g], float(case["scale"][g])
        lists = [torch.from_numpy(np.asarray(l, np.int64)) for l in idx.lists]
        c, m, v, got = tc.append_block(torch.from_numpy(idx.counts), torch.from_numpy(idx.mean),
                                       torch.from_numpy(idx.variance), lists, H, torch.from_numpy(idx.center),
                                       torch.from_numpy(kf[g, H:H + N]), torch.from_numpy(W),
                                       torch.from_numpy(b), s, case["key_mean"])
        ref, act = oracle.append_index(idx, kf[g, H:H + N], W, b, s, case["key_mean"], return_act=True)
        x = (kf[g, H:H + N] - idx.center) / np.float32(s)
        block = lambda ls: [np.asarray(l)[np.asarray(l) >= H] - H for l in ls]  # noqa: E731
        moved = expect.check_memberships(block(ref.lists), block([l.numpy() for l in got]), act,
                                         N * case["key_mean"], expect.encode_error_bound(x, W, b), f"group {g}")
        if moved == 0:
            assert np.array_equal(c.numpy(), ref.counts)
            np.testing.assert_allclose(m.numpy(), ref.mean, rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(v.numpy(), ref.variance, rtol=1e-4, atol=1e-6)
