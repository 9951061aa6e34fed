"""GPU parity on the reference's trained Qwen3-8B encoders
(pretrained/Qwen3-8B, loaded by src/prismkv/weights.py:41-70; 4 units kept
in tests/golden/qwen3_8b_encoders.npz).

Trained encoders differ from the random SAEs of the other tests in what
steers the BatchTopK threshold and the bucket sizes: structured W rows
(norms 0.45-0.88) and a per-bucket bias of mixed sign (about half of the
3000 entries negative), with saved key scales of 1.13-3.65 and query scales
of 1.16-1.60.  On these tables:

  * the prefill build at H = 65536 (8 groups): centers, activations,
    memberships bit-exact against the oracle's BatchTopK on the device's own
    activations (src/prismkv/core.py:13-26, :92-103), moments against the
    oracle's summarize (:76-89);
  * the decode on the built index: route order, ids and attention against
    the oracle (:106-183);
  * a 1024-token append (:186-201): memberships, counts and the Chan-merged
    moments, then the decode again;
  * the q_activation router with each unit's saved query scale (:131-139),
    through Native8B and through the per-group prismkv.core surface;
  * a bundle written from the fixture by save_encoders and read back by
    load_encoders drives HFNative (src/prismkv/hf_reference.py:186-233).
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import bf16_to_f32, expect
from tests.golden import trained
from tests.gpu_util import bf16_bits, bf16_tensor, log, route_outputs
from tests.test_gpu_build import check_center, check_moments, check_selection
from tests.test_gpu_update import check_group

pytestmark = pytest.mark.gpu

F = 3000


def oracle_indices(op):
    return [oracle.Index(op.history, i.center.cpu().numpy(), i.counts.cpu().numpy(), i.mean.cpu().numpy(),
                         i.variance.cpu().numpy(), [l.numpy() for l in i.lists]) for i in op.export_indices()]


def decode_vs_oracle(op, q, k, v, tag):
    idx = oracle_indices(op)
    H = op.history
    out = op(q, k, v)
    torch.cuda.synchronize()
    assert op.decode_errors() == 0
    case = dict(H=H, T=k.shape[1] - H, q=bf16_bits(q), k=bf16_bits(k), v=bf16_bits(v), indices=idx, kind="trained")
    groups = expect.expected(case)
    identical, near = expect.compare_route(groups, *route_outputs(op))
    assert identical == 8 and near == 0
    err = expect.attention_errors(bf16_bits(out), expect.expected_attention(case, groups))
    log(f"  {tag}: route identical for {identical} groups, unique {op.count.cpu().tolist()}, {err}")
    assert err["rel_l2"] <= 2e-3 and err["max_abs"] < 0.05, err
    return idx


def test_trained_build_append_decode_64k():
    from prismkv_amd import Native8B
    fx = trained.load()
    W, b, ks, _, units = trained.group_tables(fx)
    H, N, T = 65536, 1024, 64
    k = trained.mixture_keys(H + N + T, ks, seed=301)
    gen = torch.Generator(device="cuda").manual_seed(302)
    v = torch.randn(8, H + N + T, 128, generator=gen, device="cuda").to(torch.bfloat16)
    q = torch.randn(8, 4, 128, generator=gen, device="cuda").to(torch.bfloat16)
    log(f"trained build: H={H} units {units.tolist()} key scales {ks.tolist()}")
    op = Native8B.from_keys(k, H, torch.from_numpy(W), torch.from_numpy(b), torch.from_numpy(ks), 8,
                            capacity=H + N + T, keep_activations=True)
    torch.cuda.synchronize()
    kb = bf16_bits(k)
    case = dict(H=H, T=N + T, k=kb, W=W, b=b, scale=ks, key_mean=8)
    centers = op.center.cpu().numpy()
    got = op.export_indices()
    acts = op.build_activations()
    rows = np.random.default_rng(7).choice(H, 256, replace=False)
    for g in range(8):
        check_center(case, g, centers[g])
        kf = bf16_to_f32(kb[g, :H])
        x = (kf[rows] - centers[g]) / ks[g]
        ref_rows = oracle.sae_dense(x, W[g], b[g])
        dev_rows = acts[g, torch.from_numpy(rows).cuda()].cpu().numpy()
        err = float(np.abs(dev_rows - ref_rows).max())
        assert err <= 2e-6 * max(1.0, float(np.abs(ref_rows).max())), ("activation error", g, err)
        if g < trained.UNITS:  # each unit once: exact selection on the device's activations
            sel, _ = check_selection(case, g, acts[g].cpu().numpy(), got[g])
            assert sel == 8 * H
        check_moments(case, g, got[g])
        sizes = got[g].counts.cpu().numpy()
        log(f"  group {g}: memberships={got[g].memberships} live buckets={(sizes > 0).sum()} "
            f"largest={sizes.max()} act_err={err:.2e}")
    del acts
    old = decode_vs_oracle(op, q, k[:, :H + N + T], v[:, :H + N + T], "decode on the built index")
    # one update block of 1024 keys with the build's center (append_index)
    op.append(k, N)
    torch.cuda.synchronize()
    assert op.history == H + N
    act = op.update_activations(N).cpu().numpy()
    got2 = op.export_indices()
    case_u = dict(H=H, N=N, key_mean=8, indices=old, k=kb, W=W, b=b, scale=ks)
    for g in range(8):
        sel, moved, err = check_group(case_u, g, act[g], got2[g])
        log(f"  append group {g}: selected={sel} moved_at_tau={moved} act_err={err:.2e}")
        assert sel == 8 * N
    decode_vs_oracle(op, q, k, v, "decode after the append")


def test_trained_q_activation_native8b():
    # the q_activation router with the units' saved query scales, 8 groups
    from prismkv_amd import Native8B
    fx = trained.load()
    W, b, ks, qs, _ = trained.group_tables(fx)
    H, T = 20000, 33
    k = trained.mixture_keys(H + T, ks, seed=311)
    gen = torch.Generator(device="cuda").manual_seed(312)
    v = torch.randn(8, H + T, 128, generator=gen, device="cuda").to(torch.bfloat16)
    q = (torch.randn(8, 4, 128, generator=gen, device="cuda") * torch.from_numpy(qs).cuda()[:, None, None])
    q = q.to(torch.bfloat16)
    Wt, bt = torch.from_numpy(W), torch.from_numpy(b)
    op = Native8B.from_keys(k, H, Wt, bt, torch.from_numpy(ks), 8, capacity=H + T)
    op.set_query_encoders(Wt, bt, torch.from_numpy(qs))
    op.router = "q_activation"
    out = op(q, k, v)
    torch.cuda.synchronize()
    got = op.export_indices()
    feats, valid = op.features.cpu().numpy(), op.valid.cpu().numpy()
    raw, ids, count = op.raw.cpu().numpy(), op.ids.cpu().numpy(), op.count.cpu().numpy()
    qf = bf16_to_f32(bf16_bits(q))
    want = []
    for g in range(8):
        lists = [l.numpy() for l in got[g].lists]
        _, w_order, margin = oracle.qact_scores(qf[g], W[g], b[g], float(qs[g]), got[g].counts.cpu().numpy())
        nf = int((valid[g] > 0).sum())
        assert np.array_equal(feats[g][:nf], w_order), (g, margin)
        w_ids, w_meta = oracle.select_buckets(w_order, lists, H, None)
        assert feats[g][:nf].tolist() == w_meta["features"] and int(raw[g]) == w_meta["raw"], g
        assert np.array_equal(ids[g][:count[g]].astype(np.int64), w_ids), g
        want.append(dict(ids=w_ids))
        log(f"  group {g}: {nf} buckets (margin {margin:.2e}), unique {count[g]}")
    c2 = dict(H=H, T=T, q=bf16_bits(q), k=bf16_bits(k), v=bf16_bits(v), indices=oracle_indices(op), kind="qact")
    err = expect.attention_errors(bf16_bits(out), expect.expected_attention(c2, want))
    log(f"  trained q_activation decode {err}")
    assert err["rel_l2"] <= 2e-3 and err["max_abs"] < 0.05, err


@pytest.mark.parametrize("unit", range(trained.UNITS))
def test_trained_core_surface(unit):
    # one group through prismkv.core with the unit's SharedSAE and saved scales
    from prismkv_amd import core
    from prismkv_amd.weights import SharedSAE
    fx = trained.load()
    sae = SharedSAE()
    with torch.no_grad():
        sae.W_enc.copy_(torch.from_numpy(fx["W_enc"][unit]))
        sae.b_enc.copy_(torch.from_numpy(fx["b_enc"][unit]))
    ks, qs = float(fx["key_scale"][unit]), float(fx["query_scale"][unit])
    H, N, T = 3000, 500, 7
    k = trained.mixture_keys(H + N + T, np.array([ks], np.float32), seed=320 + unit)[0]
    gen = torch.Generator(device="cuda").manual_seed(330 + unit)
    v = torch.randn(H + N + T, 128, generator=gen, device="cuda").to(torch.bfloat16)
    q = torch.randn(4, 128, generator=gen, device="cuda").to(torch.bfloat16)
    kf, vf, qf = (bf16_to_f32(bf16_bits(t)) for t in (k, v, q))
    W, b = fx["W_enc"][unit], fx["b_enc"][unit]
    idx = core.build_index(k[:H], sae, ks)
    ref = oracle.build_index(kf[:H], W, b, np.float32(ks), 8, center=idx.center.cpu().numpy())
    x = (kf[:H] - idx.center.cpu().numpy()) / np.float32(ks)
    act = oracle.sae_dense(x, W, b)
    moved = expect.check_memberships(ref.lists, [l.cpu().numpy() for l in idx.lists], act, 8 * H,
                                     expect.encode_error_bound(x, W, b), f"unit {unit} build")
    idx2 = core.append_index(idx, k[H:H + N], sae, ks)
    assert idx2.history == H + N and torch.equal(idx2.center, idx.center)
    for router, kwargs in (("moments", {}), ("q_activation", dict(sae=sae, query_scale=qs))):
        score, order = core.bucket_scores(q, idx2, router=router, **kwargs)
        lists = [l.cpu().numpy() for l in idx2.lists]
        if router == "moments":
            w_score, w_order, margin, _ = oracle.bucket_scores(qf, idx2.counts.cpu().numpy(),
                                                               idx2.mean.cpu().numpy(), idx2.variance.cpu().numpy())
        else:
            w_score, w_order, margin = oracle.qact_scores(qf, W, b, np.float32(qs), idx2.counts.cpu().numpy())
        assert np.array_equal(order.cpu().numpy(), w_order), (router, margin)
        ids, meta = core.select_buckets(q, idx2, router=router, **kwargs)
        w_ids, w_meta = oracle.select_buckets(w_order, lists, H + N, None)
        assert np.array_equal(ids.cpu().numpy(), w_ids) and meta["raw"] == w_meta["raw"], router
        out = core.attend(q, k, v, ids, H + N)
        err = expect.attention_errors(bf16_bits(out), oracle.attend(qf, kf, vf, w_ids, H + N))
        log(f"  unit {unit} ({fx['unit_file'][unit]}) {router}: {len(w_order)} buckets, unique {len(w_ids)}, "
            f"build memberships moved at tau {moved}, {err}")
        assert err["rel_l2"] <= 2e-3 and err["max_abs"] < 0.05, err


def test_trained_bundle_through_hf(tmp_path):
    # the fixture written as a bundle (save_encoders) and read back
    # (load_encoders, sha256-checked) drives the model hook for two layers
    from transformers import DynamicCache
    from prismkv_amd.hf import HFNative
    from prismkv_amd.weights import Encoder, SharedSAE, load_encoders, save_encoders
    from tests.test_gpu_hf import Capture, check_call, tiny_qwen3
    fx = trained.load()
    encs = {}
    for layer in range(2):
        for g in range(8):
            u = (layer * 8 + g) % trained.UNITS
            sae = SharedSAE()
            with torch.no_grad():
                sae.W_enc.copy_(torch.from_numpy(fx["W_enc"][u]))
                sae.b_enc.copy_(torch.from_numpy(fx["b_enc"][u]))
            encs[(layer, g)] = Encoder(sae, float(fx["key_scale"][u]), float(fx["query_scale"][u]))
    save_encoders(encs, tmp_path / "bundle")
    loaded, manifest = load_encoders(tmp_path / "bundle")
    assert len(loaded) == 16 and manifest["schema"] == 1
    model = tiny_qwen3(2)
    session = HFNative(model, loaded, update_interval=256)
    cap = Capture(session)
    P, steps = 1200, 2
    ids = torch.randint(0, 256, (1, P + steps), generator=torch.Generator().manual_seed(9)).cuda()
    cache = DynamicCache(config=model.config)
    with torch.no_grad():
        model(ids[:, :P], past_key_values=cache, use_cache=True)
        for s in range(steps):
            model(ids[:, P + s:P + s + 1], past_key_values=cache, use_cache=True)
            torch.cuda.synchronize()
            for layer, q, K, V, out in cap.calls:
                err = check_call(session.ops[layer], layer, q, K, V, out)
                log(f"  step {s} layer {layer}: {err}")
            cap.calls.clear()
    session.close()
