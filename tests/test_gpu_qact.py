"""GPU parity of the q_activation router (src/prismkv/core.py:131-139)
against the oracle: the 4 queries' top-16 SAE activations, normalised per
query, scattered into bucket scores; every live bucket of positive score (up
to 64) in score order, then the union of their lists and attention.

The device's order must equal the oracle's unless the oracle's own margin
(the smallest relative gap between a query's 16th and 17th activation, or
between consecutive ordered scores) is within fp32 rounding; ids / raw /
features of the walk over the device's order are bit-exact; attention
relL2 <= 2e-3.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import bf16_to_f32, cases, expect
from tests.gpu_util import bf16_bits, bf16_tensor, log

pytestmark = pytest.mark.gpu


def check_order(got, want, margin, tag):
    same = np.array_equal(got, want)
    log(f"  {tag}: {len(got)} buckets, order identical={same}, margin={margin:.2e}")
    assert same, (tag, np.asarray(got).tolist(), np.asarray(want).tolist(), margin)
    return same


@pytest.mark.parametrize("cap", [None, 0.05])
def test_core_q_activation(cap):
    from prismkv_amd import core
    from tests.test_gpu_core import sae
    H = 4096
    case = cases.build_case("random", H=H, T=9, seed=211)
    k, v, q = bf16_tensor(case["k"][0]), bf16_tensor(case["v"][0]), bf16_tensor(case["q"][0])
    enc = sae(8, bias=0.05)
    idx = core.build_index(k[:H], enc, 1.0)
    qf = bf16_to_f32(case["q"][0])
    W, b = enc.W_enc.detach().numpy(), enc.b_enc.detach().numpy()
    score, order = core.bucket_scores(q, idx, router="q_activation", sae=enc, query_scale=2.0)
    w_score, w_order, margin = oracle.qact_scores(qf, W, b, 2.0, idx.counts.cpu().numpy())
    o = order.cpu().numpy()
    check_order(o, w_order, margin, "order")
    assert np.allclose(score.cpu().numpy(), w_score, rtol=1e-4, atol=1e-7)
    ids, meta = core.select_buckets(q, idx, unique_cap=cap, router="q_activation", sae=enc, query_scale=2.0)
    w_ids, w_meta = oracle.select_buckets(o, [l.cpu().numpy() for l in idx.lists], H, cap)
    assert np.array_equal(ids.cpu().numpy(), w_ids)
    for key in ("features", "raw", "unique", "limit", "candidate_buckets"):
        assert meta[key] == w_meta[key], key
    out = core.attend(q, k, v, ids, H)
    err = expect.attention_errors(bf16_bits(out), oracle.attend(qf, bf16_to_f32(case["k"][0]),
                                                                bf16_to_f32(case["v"][0]), w_ids, H))
    log(f"  cap={cap}: {len(o)} candidates, unique={meta['unique']} raw={meta['raw']} {err}")
    assert err["rel_l2"] <= 2e-3 and err["max_abs"] < 0.05, err


@pytest.mark.parametrize("cap", [None, 0.02])
def test_native8b_q_activation(cap):
    # 8 groups through Native8B: route (up to 64 buckets) + union + attention
    from prismkv_amd import Native8B
    H, T = 20000, 17
    case = cases.build_case("random", H=H, T=T, seed=221)
    k, v, q = bf16_tensor(case["k"]), bf16_tensor(case["v"]), bf16_tensor(case["q"])
    W, b, scale = (torch.from_numpy(case[x]) for x in ("W", "b", "scale"))
    op = Native8B.from_keys(k, H, W, b, scale, 8, capacity=H + T, unique_cap=cap)
    qscale = np.array([0.5 + 0.1 * g for g in range(8)], np.float32)
    op.set_query_encoders(W, b, torch.from_numpy(qscale))
    op.router = "q_activation"
    out = op(q, k, v)
    torch.cuda.synchronize()
    assert op.features.shape == (8, 64)
    got = op.export_indices()
    feats, valid = op.features.cpu().numpy(), op.valid.cpu().numpy()
    raw, ids, count = op.raw.cpu().numpy(), op.ids.cpu().numpy(), op.count.cpu().numpy()
    qf = bf16_to_f32(case["q"])
    want = []
    for g in range(8):
        lists = [l.numpy() for l in got[g].lists]
        _, w_order, margin = oracle.qact_scores(qf[g], case["W"][g], case["b"][g], float(qscale[g]),
                                                got[g].counts.cpu().numpy())
        nf = int((valid[g] > 0).sum())
        if cap is None:
            check_order(feats[g][:nf], w_order, margin, f"group {g}")
            order = feats[g][:nf]
        else:
            order = w_order  # the device's pre-cap order is not kept; the walk runs over the oracle's
        w_ids, w_meta = oracle.select_buckets(order, lists, H, cap)
        assert feats[g][:nf].tolist() == w_meta["features"] and int(raw[g]) == w_meta["raw"], (g, margin)
        assert np.array_equal(ids[g][:count[g]].astype(np.int64), w_ids), g
        want.append(dict(ids=ids[g][:count[g]].astype(np.int64)))
    idx = [oracle.Index(H, i.center.cpu().numpy(), i.counts.cpu().numpy(), i.mean.cpu().numpy(),
                        i.variance.cpu().numpy(), [l.numpy() for l in i.lists]) for i in got]
    c2 = dict(H=H, T=T, q=case["q"], k=case["k"], v=case["v"], indices=idx, kind="qact")
    err = expect.attention_errors(bf16_bits(out), expect.expected_attention(c2, want))
    log(f"  cap={cap}: buckets {[int((x > 0).sum()) for x in valid]} unique {count.tolist()} {err}")
    assert err["rel_l2"] <= 2e-3 and err["max_abs"] < 0.05, err
    # back to moments: the fused path and [8,16] selections again
    op.router = "moments"
    op.unique_cap = None
    op(q, k, v)
    assert op.features.shape == (8, 16) and op.decode_errors() == 0


def test_hf_q_activation_decode():
    from prismkv_amd.hf import HFNative
    from tests.test_gpu_hf import Capture, encoders, tiny_qwen3
    from transformers import DynamicCache
    model = tiny_qwen3(1)
    enc = encoders(1, seed=13)
    for e in enc.values():
        e.query_scale = 0.8
    session = HFNative(model, enc, router="q_activation")
    cap = Capture(session)
    P = 700
    ids = torch.randint(0, 256, (1, P + 2), generator=torch.Generator().manual_seed(4)).cuda()
    cache = DynamicCache(config=model.config)
    with torch.no_grad():
        model(ids[:, :P], past_key_values=cache, use_cache=True)
        model(ids[:, P:P + 1], past_key_values=cache, use_cache=True)
    torch.cuda.synchronize()
    layer, q, K, V, out = cap.calls[-1]
    op = session.ops[layer]
    got = op.export_indices()
    qf = bf16_to_f32(bf16_bits(q))
    want = []
    for g in range(8):
        W = enc[(layer, g)].sae.W_enc.detach().numpy()
        b = enc[(layer, g)].sae.b_enc.detach().numpy()
        _, w_order, margin = oracle.qact_scores(qf[g], W, b, 0.8, got[g].counts.cpu().numpy())
        w_ids, _ = oracle.select_buckets(w_order, [l.numpy() for l in got[g].lists], P, None)
        dev = op.features[g][op.valid[g] > 0].cpu().numpy()
        if check_order(dev, w_order, margin, f"group {g}"):
            assert np.array_equal(op.ids[g][:op.count[g]].cpu().numpy().astype(np.int64), w_ids)
        want.append(dict(ids=op.ids[g][:op.count[g]].cpu().numpy().astype(np.int64)))
    idx = [oracle.Index(P, i.center.cpu().numpy(), i.counts.cpu().numpy(), i.mean.cpu().numpy(),
                        i.variance.cpu().numpy(), [l.numpy() for l in i.lists]) for i in got]
    c2 = dict(H=P, T=K.shape[1] - P, q=bf16_bits(q), k=bf16_bits(K), v=bf16_bits(V), indices=idx, kind="qact")
    err = expect.attention_errors(bf16_bits(out), expect.expected_attention(c2, want))
    log(f"  hf q_activation decode: {err}")
    assert err["rel_l2"] <= 2e-3 and err["max_abs"] < 0.05, err
    session.close()
