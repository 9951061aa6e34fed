"""GPU parity of the prismkv.core surface (prismkv_amd.core, the counterpart
of src/prismkv/core.py) against the CPU oracle, one KV group at a time at the
native geometry (head_dim 128, F = 3000, 4 query heads):

  * positive_global_topk: bit-exact flat indices, in the reference's order
    (strict values ascending, then ties ascending), on matrices steering every
    branch of core.py:13-26 (distinct values, negative values, ties that
    overflow the budget, fewer positives than the budget, an empty budget, a
    budget beyond the matrix);
  * build_index / append_index / summarize: lists equal to the oracle's
    (or different only within rounding of the threshold), counts exact,
    moments within fp32 rounding, the center the exact mean;
  * bucket_scores / select_buckets: the device order equals the oracle's
    (near-ties aside), scores within fp32 rounding, ids / raw / features of the
    walk bit-exact, with and without a unique cap;
  * attend: relative L2 <= 2e-3 against fp64.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import bf16_to_f32, cases, expect
from tests.gpu_util import bf16_bits, bf16_tensor, log

pytestmark = pytest.mark.gpu

F = 3000


def sae(seed, bias=0.0):
    from prismkv_amd.weights import SharedSAE
    s = SharedSAE()
    with torch.no_grad():
        s.W_enc.copy_(torch.randn(F, 128, generator=torch.Generator().manual_seed(seed)) / 128 ** 0.5)
        s.b_enc.fill_(bias)
    return s


@pytest.mark.parametrize("kind", ["random", "signed", "ties", "few", "empty_budget", "big_budget", "bf16",
                                  "crowded", "wide_bin"])
def test_positive_global_topk(kind):
    from prismkv_amd import core
    gen = torch.Generator(device="cuda").manual_seed(3)
    N = 257
    a = torch.randn(N, F, generator=gen, device="cuda")
    count = 8 * N
    if kind == "crowded":
        # 2048 values in [10, 11) (one first-digit bin, tau's) at flat indices
        # [0, 1024) and [262144, 263168): the positions one refine workgroup
        # reads, so its 1024-entry candidate buffer overflows into the list
        a = a.abs() * 0.01
        flat = a.view(-1)
        big = 10.0 + torch.rand(2048, generator=gen, device="cuda")
        flat[:1024] = big[:1024]
        flat[262144:263168] = big[1024:]
        count = 1500
    elif kind == "wide_bin":
        # 600000 positive values in tau's first-digit bin: more candidates than
        # the compact list holds (2^19 entries less the chunk tails' 2^18 at
        # this block size), so the later passes scan every value
        a = 1.0 + torch.rand(N, F, generator=gen, device="cuda") * 0.0625
        a.view(-1)[600000:] = -1.0
        count = 5000
    if kind == "random":
        a = a.relu()
    elif kind == "ties":
        a = (a > 0.5).float() * 0.75  # 0.75 ties far beyond the budget
    elif kind == "few":
        a = torch.where(a > 3.0, a, torch.zeros_like(a))  # fewer positives than the budget
    elif kind == "empty_budget":
        count = 0
    elif kind == "big_budget":
        count = N * F + 5
    elif kind == "bf16":
        a = a.relu().to(torch.bfloat16)
    got = core.positive_global_topk(a, count).cpu().numpy()
    want = oracle.positive_global_topk(a.float().cpu().numpy(), count)
    log(f"  {kind}: {len(got)} selected")
    assert np.array_equal(got, want), (kind, len(got), len(want))


def index_inputs(H, seed):
    case = cases.build_case("random", H=H, T=8, seed=seed)
    return case, bf16_tensor(case["k"][0])


def test_build_and_summarize():
    from prismkv_amd import core
    H = 1500
    case, k = index_inputs(H, 171)
    enc = sae(5)
    idx = core.build_index(k[:H], enc, 1.25)
    kf = bf16_to_f32(case["k"][0, :H])
    exact = kf.astype(np.float64).mean(0)
    c = idx.center.cpu().numpy()
    assert (np.abs(c - exact) <= np.spacing(np.abs(exact).astype(np.float32))).all()
    ref = oracle.build_index(kf, enc.W_enc.detach().numpy(), enc.b_enc.detach().numpy(), 1.25, 8, center=c)
    act = oracle.sae_dense((kf - c) / np.float32(1.25), enc.W_enc.detach().numpy(), enc.b_enc.detach().numpy())
    x = (kf - c) / np.float32(1.25)
    moved = expect.check_memberships(ref.lists, [l.cpu().numpy() for l in idx.lists], act, 8 * H,
                                     expect.encode_error_bound(x, enc.W_enc.detach().numpy(),
                                                               enc.b_enc.detach().numpy()), "build")
    log(f"  build: {idx.memberships} memberships, {moved} differing from the oracle (within rounding of tau)")
    assert idx.history == H and idx.counts.dtype == torch.long
    # summarize over the device lists, with and without a center
    c2, m2, v2 = oracle.summarize(kf, [l.cpu().numpy() for l in idx.lists])
    assert np.array_equal(idx.counts.cpu().numpy(), c2)
    assert np.allclose(idx.mean.cpu().numpy(), m2, rtol=1e-6, atol=1e-7)
    assert np.allclose(idx.variance.cpu().numpy(), v2, rtol=1e-6, atol=1e-7)
    s = core.summarize(k[:H], idx.lists)
    assert torch.equal(s.mean, idx.mean) and torch.equal(s.variance, idx.variance) and torch.equal(s.center,
                                                                                                   idx.center)
    s2 = core.summarize(k[:H], idx.lists, center=torch.zeros(128))
    assert torch.equal(s2.mean, idx.mean) and torch.equal(s2.center, torch.zeros(128))


def test_append_index():
    from prismkv_amd import core
    H, N = 900, 300
    case, k = index_inputs(H + N, 181)
    enc = sae(6)
    idx = core.build_index(k[:H], enc, 1.5)
    nxt = core.append_index(idx, k[H:H + N], enc, 1.5)
    assert nxt.history == H + N and idx.history == H
    kf = bf16_to_f32(case["k"][0])
    o0 = oracle.Index(H, idx.center.cpu().numpy(), idx.counts.cpu().numpy(), idx.mean.cpu().numpy(),
                      idx.variance.cpu().numpy(), [l.cpu().numpy() for l in idx.lists])
    o1, act = oracle.append_index(o0, kf[H:H + N], enc.W_enc.detach().numpy(), enc.b_enc.detach().numpy(), 1.5, 8,
                                  return_act=True)
    same = all(np.array_equal(a.cpu().numpy(), b) for a, b in zip(nxt.lists, o1.lists))
    from tests.test_gpu_build import block_lists
    x = (kf[H:H + N] - idx.center.cpu().numpy()) / np.float32(1.5)
    moved = expect.check_memberships(block_lists(o1.lists, H, N), block_lists([l.cpu() for l in nxt.lists], H, N),
                                     act, 8 * N, expect.encode_error_bound(x, enc.W_enc.detach().numpy(),
                                                                           enc.b_enc.detach().numpy()), "append")
    log(f"  append: lists identical={same}, block memberships differing (within rounding of tau): {moved}")
    if same:
        assert np.array_equal(nxt.counts.cpu().numpy(), o1.counts)
        assert np.allclose(nxt.mean.cpu().numpy(), o1.mean, rtol=1e-5, atol=1e-6)
        assert np.allclose(nxt.variance.cpu().numpy(), o1.variance, rtol=1e-5, atol=1e-6)
    # the source index is untouched and still routes as before
    assert len(idx.lists[0]) == len(o0.lists[0])


@pytest.mark.parametrize("cap", [None, 0.05])
def test_scores_selection_and_attention(cap):
    from prismkv_amd import core
    H, T = 4096, 7
    case, k = index_inputs(H, 191)
    v = bf16_tensor(case["v"][0])
    q = bf16_tensor(case["q"][0])
    idx = core.build_index(k[:H], sae(7), 1.0)
    lists = [l.cpu().numpy() for l in idx.lists]
    qf = bf16_to_f32(case["q"][0])
    score, order = core.bucket_scores(q, idx)
    w_score, w_order, margin, ties = oracle.bucket_scores(qf, idx.counts.cpu().numpy(), idx.mean.cpu().numpy(),
                                                          idx.variance.cpu().numpy())
    o = order.cpu().numpy()
    log(f"  order identical={np.array_equal(o, w_order)} margin={margin:.2e}")
    assert np.array_equal(o, w_order), (o.tolist(), w_order.tolist(), margin)
    assert np.allclose(score.cpu().numpy(), w_score, rtol=1e-5, atol=1e-9)
    ids, meta = core.select_buckets(q, idx, unique_cap=cap)
    w_ids, w_meta = oracle.select_buckets(o, lists, H, cap)
    assert np.array_equal(ids.cpu().numpy(), w_ids)
    for key in ("features", "raw", "unique", "limit", "candidate_buckets"):
        assert meta[key] == w_meta[key], key
    assert torch.equal(meta["scores"], score)
    out = core.attend(q, k, v, ids, H)
    want = oracle.attend(qf, bf16_to_f32(case["k"][0]), bf16_to_f32(case["v"][0]), w_ids, H)
    err = expect.attention_errors(bf16_bits(out), want)
    log(f"  cap={cap}: unique={meta['unique']} raw={meta['raw']} {err}")
    assert err["rel_l2"] <= 2e-3 and err["max_abs"] < 0.05, err
    assert out.dtype == torch.bfloat16 and out.shape == (4, 128)


def test_attend_edges():
    from prismkv_amd import core
    case, k = index_inputs(64, 201)
    v = bf16_tensor(case["v"][0])
    q = bf16_tensor(case["q"][0])
    empty = torch.zeros(0, dtype=torch.long, device="cuda")
    # no history rows and no tail: zeros (core.py:179-180)
    assert torch.equal(core.attend(q, k[:64], v[:64], empty, 64), torch.zeros_like(q))
    # tail only, and unsorted history ids
    for ids, H in ((empty, 60), (torch.tensor([40, 3, 17], device="cuda"), 60)):
        out = core.attend(q, k[:72], v[:72], ids, H)
        want = oracle.attend(bf16_to_f32(case["q"][0]), bf16_to_f32(case["k"][0, :72]), bf16_to_f32(case["v"][0, :72]),
                             ids.cpu().numpy(), H)
        err = expect.attention_errors(bf16_bits(out), want)
        assert err["rel_l2"] <= 2e-3, err
