"""GPU checks of the native Hugging Face decode backend (prismkv_amd.hf,
the counterpart of src/prismkv/hf_reference.py) on a small random-init
Qwen3 with the 8B attention geometry (32 query heads, 8 KV heads, d = 128):

  * every decode step's attention output of every layer equals the oracle's
    route + attention (src/prismkv/core.py:106-183) over the index the device
    holds at that step, given the step's own Q/K/V;
  * the index history follows the reference's update trigger
    (src/prismkv/hf_reference.py:205-211) step by step, with capacity growth;
  * the dense control (mode "all_read") leaves the model's logits unchanged.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import expect
from tests.gpu_util import bf16_bits, log

pytestmark = pytest.mark.gpu


def tiny_qwen3(layers):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=16384)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(3)
    return Qwen3ForCausalLM(cfg).to(device="cuda", dtype=torch.bfloat16).eval()


def encoders(layers, seed=11):
    from prismkv_amd.weights import Encoder, SharedSAE
    gen = torch.Generator().manual_seed(seed)
    out = {}
    for l in range(layers):
        for g in range(8):
            sae = SharedSAE()
            with torch.no_grad():
                sae.W_enc.copy_(torch.randn(3000, 128, generator=gen) / 128 ** 0.5)
            out[(l, g)] = Encoder(sae, 1.0, 1.0)
    return out


class Capture:
    """Wraps the session's forward to keep each decode call's Q/K/V and output."""

    def __init__(self, session):
        self.session, self.calls = session, []
        self._forward = session.forward
        session.forward = self

    def __call__(self, module, q, k, v, mask, **kw):
        out = self._forward(module, q, k, v, mask, **kw)
        if q.shape[-2] == 1 and module.layer_idx in self.session.ops:
            self.calls.append((module.layer_idx, q[0, :, 0].reshape(8, 4, 128).clone(), k[0].clone(), v[0].clone(),
                               out[0].reshape(8, 4, 128).clone()))
        return out


def check_call(op, layer, q, K, V, out):
    H = op.history
    idx = [oracle.Index(H, i.center.cpu().numpy(), i.counts.cpu().numpy(), i.mean.cpu().numpy(),
                        i.variance.cpu().numpy(), [l.numpy() for l in i.lists]) for i in op.export_indices()]
    case = dict(H=H, T=K.shape[1] - H, q=bf16_bits(q), k=bf16_bits(K), v=bf16_bits(V), indices=idx, kind="hf")
    groups = expect.expected(case)
    err = expect.attention_errors(bf16_bits(out), expect.expected_attention(case, groups))
    assert op.decode_errors() == 0
    assert err["rel_l2"] <= 2e-3 and err["max_abs"] < 0.05, (layer, err)
    return err


def test_decode_steps_match_the_oracle():
    from prismkv_amd.hf import HFNative
    layers, P, steps = 2, 1500, 3
    model = tiny_qwen3(layers)
    session = HFNative(model, encoders(layers), update_interval=64)
    cap = Capture(session)
    ids = torch.randint(0, 256, (1, P + steps), generator=torch.Generator().manual_seed(1)).cuda()
    from transformers import DynamicCache
    cache = DynamicCache(config=model.config)
    with torch.no_grad():
        model(ids[:, :P], past_key_values=cache, use_cache=True)
        for s in range(steps):
            model(ids[:, P + s:P + s + 1], past_key_values=cache, use_cache=True)
            torch.cuda.synchronize()
            for layer, q, K, V, out in cap.calls:
                err = check_call(session.ops[layer], layer, q, K, V, out)
                log(f"  step {s} layer {layer}: history={session.ops[layer].history} tail={K.shape[1] - session.ops[layer].history} {err}")
            cap.calls.clear()
    recs = session.records
    assert len(recs) == layers * 8 * steps
    assert all(r["history"] == P and r["unique"] > 0 and r["buckets"] == 16 for r in recs)
    session.close()


def test_update_trigger_and_growth():
    from prismkv_amd.hf import HFNative
    layers, P, steps, interval = 1, 300, 40, 16
    model = tiny_qwen3(layers)
    session = HFNative(model, encoders(layers, seed=12), update_interval=interval, capacity_step=16)
    cap = Capture(session)
    ids = torch.randint(0, 256, (1, P + steps), generator=torch.Generator().manual_seed(2)).cuda()
    from transformers import DynamicCache
    cache = DynamicCache(config=model.config)
    h = P
    with torch.no_grad():
        model(ids[:, :P], past_key_values=cache, use_cache=True)
        for s in range(steps):
            model(ids[:, P + s:P + s + 1], past_key_values=cache, use_cache=True)
            total = P + s + 1
            while total - h > interval:  # src/prismkv/hf_reference.py:209
                h += interval
            op = session.ops[0]
            assert op.history == h, (s, op.history, h)
            assert op.capacity >= total
            if s in (0, 17, steps - 1):
                torch.cuda.synchronize()
                layer, q, K, V, out = cap.calls[-1]
                err = check_call(op, layer, q, K, V, out)
                log(f"  step {s}: history={op.history} capacity={op.capacity} {err}")
            cap.calls.clear()
    assert [r["history"] for r in session.records][-1] == h
    session.close()


def test_all_read_is_the_dense_model():
    from prismkv_amd.hf import HFNative
    model = tiny_qwen3(1)
    ids = torch.randint(0, 256, (1, 200), generator=torch.Generator().manual_seed(3)).cuda()
    from transformers import DynamicCache

    def run():
        cache = DynamicCache(config=model.config)
        with torch.no_grad():
            model(ids[:, :190], past_key_values=cache, use_cache=True)
            return [model(ids[:, t:t + 1], past_key_values=cache, use_cache=True).logits for t in range(190, 200)]
    dense = run()
    session = HFNative(model, encoders(1), mode="all_read")
    control = run()
    session.close()
    for a, b in zip(dense, control):
        assert torch.equal(a, b)
    assert all(r["unique"] == 190 for r in session.records)


def test_detailed_records_match_the_oracle():
    # detailed_records=True adds initial_history, old_unique, old_raw and the
    # generated_indexed_* fields (src/prismkv/hf_reference.py:216-231); after
    # update blocks some selected ids lie beyond the prefix, so the generated
    # fields are nonzero.  Checked against the oracle's walk over the device's
    # kept buckets on the index the device holds.
    from prismkv_amd.hf import HFNative
    from transformers import DynamicCache
    layers, P, steps, interval = 1, 600, 70, 32
    model = tiny_qwen3(layers)
    session = HFNative(model, encoders(layers, seed=21), update_interval=interval, detailed_records=True)
    ids = torch.randint(0, 256, (1, P + steps), generator=torch.Generator().manual_seed(5)).cuda()
    cache = DynamicCache(config=model.config)
    generated = 0
    with torch.no_grad():
        model(ids[:, :P], past_key_values=cache, use_cache=True)
        for s in range(steps):
            model(ids[:, P + s:P + s + 1], past_key_values=cache, use_cache=True)
            if s in (0, steps - 1):
                op = session.ops[0]
                recs = session.records[-8:]
                got = op.export_indices()
                feats, valid = op.features.cpu().numpy(), op.valid.cpu().numpy()
                for g, rec in enumerate(recs):
                    kept = [int(f) for f, ok in zip(feats[g], valid[g]) if ok > 0]
                    lists = [l.numpy() for l in got[g].lists]
                    w_ids, meta = oracle.select_buckets(np.array(kept, np.int64), lists, op.history, None)
                    old_unique = int((w_ids < P).sum())
                    old_raw = sum(int((lists[b] < P).sum()) for b in kept)
                    assert rec["initial_history"] == P and rec["unique"] == len(w_ids) and rec["raw"] == meta["raw"]
                    assert rec["old_unique"] == old_unique and rec["old_raw"] == old_raw, (s, g, rec)
                    assert rec["generated_indexed_unique"] == len(w_ids) - old_unique
                    assert rec["generated_indexed_raw"] == meta["raw"] - old_raw
                    generated += rec["generated_indexed_unique"]
                log(f"  step {s}: history={op.history}, generated ids selected {[r['generated_indexed_unique'] for r in recs]}")
    assert session.ops[0].history > P and generated > 0
    session.close()
