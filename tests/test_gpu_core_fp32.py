"""The prismkv.core surface on fp32 inputs.

The reference's core computes on `.float()` of inputs of any float dtype
(src/prismkv/core.py:92-103,106-139,170-183) and its replay example runs it on
fp32 tensors (examples/replay.py:15-21).  Here the replay shape -- 8 KV groups
x 4 query heads, d = 128, F = 3000, H = 1024 history + 32 tail, Top-16, keys /
queries / values iid N(0, 1) in fp32, W ~ N(0, 1/128), b = 0 -- goes through
build_index, bucket_scores, select_buckets and attend at fp32 (the `_f32`
entry points), against the oracle on the same fp32 values:

  * build_index: the center is the mean to fp32 rounding, the lists equal the
    oracle's (or differ only within rounding of the BatchTopK threshold), the
    counts are exact and the moments agree to fp32 rounding;
  * the route order equals the oracle's and the union's ids are bit-exact;
  * attend (fp32 q / K / V, fp32 output) is within relative L2 1e-5 of fp64,
    a hundredth of what bf16 rounding of the inputs alone costs: the rows are
    read at full precision;
  * append_index and summarize of fp32 blocks, q_activation routing of fp32
    queries, fp16 keys (widened exactly) and a mixed bf16 / fp32 attend.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import bf16_to_f32, cases, expect, f32_to_bf16
from tests.gpu_util import log

pytestmark = pytest.mark.gpu

H, T = 1024, 32


def encoder(W, b):
    from prismkv_amd.weights import SharedSAE
    s = SharedSAE()
    with torch.no_grad():
        s.W_enc.copy_(torch.from_numpy(W))
        s.b_enc.copy_(torch.from_numpy(b))
    return s


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.fixture(scope="module")
def replay():
    return cases.replay_case(seed=5, H=H, T=T, bf16=False)


def check_index(idx, keys, W, b, scale, tag):
    """Device build of fp32 `keys` vs the oracle on the same values."""
    c = idx.center.cpu().numpy()
    exact = keys.astype(np.float64).mean(0)
    assert (np.abs(c - exact) <= np.spacing(np.abs(exact).astype(np.float32))).all(), tag
    ref = oracle.build_index(keys, W, b, scale, 8, center=c)
    x = (keys - c) / np.float32(scale)
    act = oracle.sae_dense(x, W, b)
    lists = [l.cpu().numpy() for l in idx.lists]
    moved = expect.check_memberships(ref.lists, lists, act, 8 * len(keys), expect.encode_error_bound(x, W, b), tag)
    counts, mean, var = oracle.summarize(keys, lists)
    assert np.array_equal(idx.counts.cpu().numpy(), counts), tag
    assert np.allclose(idx.mean.cpu().numpy(), mean, rtol=1e-6, atol=1e-7), tag
    assert np.allclose(idx.variance.cpu().numpy(), var, rtol=1e-6, atol=1e-7), tag
    return moved


def test_replay_shape_at_fp32(replay):
    from prismkv_amd import core
    errs, bf16_cost = [], []
    for g in range(8):
        W, b = cases.sae_weights(5, g)
        enc = encoder(W, b)
        k, v, q = (torch.from_numpy(replay[x][g]).cuda() for x in ("k", "v", "q"))
        assert k.dtype == torch.float32
        idx = core.build_index(k[:H], enc, 1.0)
        moved = check_index(idx, replay["k"][g, :H], W, b, 1.0, f"group {g}")
        # the oracle's own index of the replay case (built on the same fp32 keys)
        same = all(np.array_equal(a.cpu().numpy(), o) for a, o in zip(idx.lists, replay["indices"][g].lists))
        score, order = core.bucket_scores(q, idx)
        w_score, w_order, margin, _ = oracle.bucket_scores(replay["q"][g], idx.counts.cpu().numpy(),
                                                           idx.mean.cpu().numpy(), idx.variance.cpu().numpy())
        o = order.cpu().numpy()
        assert np.array_equal(o, w_order), (g, o.tolist(), w_order.tolist(), margin)
        assert np.allclose(score.cpu().numpy(), w_score, rtol=1e-5, atol=1e-9)
        ids, meta = core.select_buckets(q, idx)
        w_ids, w_meta = oracle.select_buckets(o, [l.cpu().numpy() for l in idx.lists], H, None)
        assert np.array_equal(ids.cpu().numpy(), w_ids)
        for key in ("features", "raw", "unique", "limit", "candidate_buckets"):
            assert meta[key] == w_meta[key], key
        out = core.attend(q, k, v, ids, H)
        assert out.dtype == torch.float32 and out.shape == (4, 128)
        want = oracle.attend(replay["q"][g], replay["k"][g], replay["v"][g], w_ids, H)
        rounded = [bf16_to_f32(f32_to_bf16(replay[x][g])) for x in ("q", "k", "v")]
        errs.append(rel(out.cpu().numpy(), want))
        bf16_cost.append(rel(oracle.attend(*rounded, w_ids, H), want))
        log(f"  group {g}: memberships {idx.memberships} ({moved} moved, oracle index identical={same}), "
            f"unique={meta['unique']} raw={meta['raw']} relL2={errs[-1]:.2e} (bf16 inputs: {bf16_cost[-1]:.2e})")
        assert errs[-1] <= 1e-5
        assert errs[-1] <= bf16_cost[-1] / 100
    log(f"  fp32 attend relL2 max {max(errs):.2e}; bf16 rounding of the inputs alone {min(bf16_cost):.2e} or more")


def test_append_and_summarize_fp32(replay):
    from prismkv_amd import core
    W, b = cases.sae_weights(5, 1)
    enc = encoder(W, b)
    keys = replay["k"][1]
    k = torch.from_numpy(keys).cuda()
    h0 = 768
    idx = core.build_index(k[:h0], enc, 1.5)
    check_index(idx, keys[:h0], W, b, 1.5, "build")
    nxt = core.append_index(idx, k[h0:H], enc, 1.5)
    o0 = oracle.Index(h0, idx.center.cpu().numpy(), idx.counts.cpu().numpy(), idx.mean.cpu().numpy(),
                      idx.variance.cpu().numpy(), [l.cpu().numpy() for l in idx.lists])
    o1, act = oracle.append_index(o0, keys[h0:H], W, b, 1.5, 8, return_act=True)
    from tests.test_gpu_build import block_lists
    x = (keys[h0:H] - idx.center.cpu().numpy()) / np.float32(1.5)
    moved = expect.check_memberships(block_lists(o1.lists, h0, H - h0), block_lists([l.cpu() for l in nxt.lists], h0,
                                                                                   H - h0),
                                     act, 8 * (H - h0), expect.encode_error_bound(x, W, b), "append")
    same = all(np.array_equal(a.cpu().numpy(), o) for a, o in zip(nxt.lists, o1.lists))
    log(f"  append of 256 fp32 keys: lists identical={same}, {moved} block memberships moved")
    if same:
        assert np.array_equal(nxt.counts.cpu().numpy(), o1.counts)
        assert np.allclose(nxt.mean.cpu().numpy(), o1.mean, rtol=1e-5, atol=1e-6)
        assert np.allclose(nxt.variance.cpu().numpy(), o1.variance, rtol=1e-5, atol=1e-6)
    # summarize of the appended lists over all H fp32 keys equals a fresh two-pass summary
    s = core.summarize(k[:H], nxt.lists, center=nxt.center)
    counts, mean, var = oracle.summarize(keys[:H], [l.cpu().numpy() for l in nxt.lists])
    assert np.array_equal(s.counts.cpu().numpy(), counts)
    assert np.allclose(s.mean.cpu().numpy(), mean, rtol=1e-6, atol=1e-7)
    assert np.allclose(s.variance.cpu().numpy(), var, rtol=1e-6, atol=1e-7)


def test_q_activation_fp32_queries(replay):
    from prismkv_amd import core
    from tests.test_gpu_qact import check_order
    W, b = cases.sae_weights(5, 2)
    b = np.full_like(b, 0.05)
    enc = encoder(W, b)
    k = torch.from_numpy(replay["k"][2]).cuda()
    q = torch.from_numpy(replay["q"][2]).cuda()
    idx = core.build_index(k[:H], enc, 1.0)
    score, order = core.bucket_scores(q, idx, router="q_activation", sae=enc, query_scale=2.0)
    w_score, w_order, margin = oracle.qact_scores(replay["q"][2], W, b, 2.0, idx.counts.cpu().numpy())
    check_order(order.cpu().numpy(), w_order, margin, "fp32 q_activation")
    assert np.allclose(score.cpu().numpy(), w_score, rtol=1e-4, atol=1e-7)


def test_fp16_keys_and_mixed_attend(replay):
    from prismkv_amd import core
    W, b = cases.sae_weights(5, 3)
    enc = encoder(W, b)
    # fp16 keys: widened exactly to fp32, so the index is the fp32 index of the fp16 values
    k16 = torch.from_numpy(replay["k"][3]).cuda().half()
    keys = k16.float().cpu().numpy()
    idx = core.build_index(k16[:H], enc, 1.0)
    check_index(idx, keys[:H], W, b, 1.0, "fp16 keys")
    # bf16 queries against fp32 K / V: computed on .float() of each, returned in q's dtype
    q = torch.from_numpy(replay["q"][3]).cuda().bfloat16()
    k, v = torch.from_numpy(replay["k"][3]).cuda(), torch.from_numpy(replay["v"][3]).cuda()
    ids = torch.arange(0, H, 3, device="cuda")
    out = core.attend(q, k, v, ids, H)
    assert out.dtype == torch.bfloat16
    want = oracle.attend(q.float().cpu().numpy(), replay["k"][3], replay["v"][3], ids.cpu().numpy(), H)
    # the fp32 result rounded to bf16: within half a bf16 step of the fp64 value (a whole step allowed)
    got = out.float().cpu().numpy().astype(np.float64)
    assert (np.abs(got - want) <= np.abs(want) * 2.0 ** -8 + 1e-6).all()
