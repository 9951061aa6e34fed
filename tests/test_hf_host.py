"""Host-side checks of the encoder bundle format (src/prismkv/weights.py:18-70)
and of the native Hugging Face session's plumbing (registration, argument
checks, prefill through the model's own attention) -- no GPU needed."""
import json

import pytest
import torch

from prismkv_amd.weights import Encoder, SharedSAE, layer_tables, load_encoders, save_encoders


def encoders(layers=1, seed=0):
    torch.manual_seed(seed)
    return {(l, g): Encoder(SharedSAE(), 1.0 + 0.5 * g, 2.0) for l in range(layers) for g in range(8)}


def test_bundle_round_trip(tmp_path):
    enc = encoders(2)
    save_encoders(enc, tmp_path / "b", metadata={"model": "tiny"})
    got, manifest = load_encoders(tmp_path / "b")
    assert manifest["schema"] == 1 and manifest["metadata"] == {"model": "tiny"}
    assert set(got) == set(enc)
    for unit, e in enc.items():
        assert torch.equal(got[unit].sae.W_enc, e.sae.W_enc) and torch.equal(got[unit].sae.b_enc, e.sae.b_enc)
        assert got[unit].key_scale == e.key_scale and got[unit].query_scale == e.query_scale
    W, b, scale, key_mean = layer_tables(got, 1)
    assert W.shape == (8, 3000, 128) and b.shape == (8, 3000) and key_mean == 8
    assert torch.equal(scale, torch.tensor([1.0 + 0.5 * g for g in range(8)]))
    with pytest.raises(FileExistsError):  # never overwrite
        save_encoders(enc, tmp_path / "b")


def test_bundle_rejects_tampering(tmp_path):
    save_encoders(encoders(1), tmp_path / "b")
    (tmp_path / "b" / "l00_g03.pt").write_bytes(b"not the saved tensors")
    with pytest.raises(ValueError, match="hash"):
        load_encoders(tmp_path / "b")
    save_encoders(encoders(1), tmp_path / "c")
    m = json.loads((tmp_path / "c" / "manifest.json").read_text())
    m["schema"] = 2
    (tmp_path / "c" / "manifest.json").write_text(json.dumps(m))
    with pytest.raises(ValueError, match="schema"):
        load_encoders(tmp_path / "c")


def test_load_keeps_the_rng_stream(tmp_path):
    save_encoders(encoders(1), tmp_path / "b")
    torch.manual_seed(7)
    want = torch.rand(3)
    torch.manual_seed(7)
    load_encoders(tmp_path / "b")
    assert torch.equal(torch.rand(3), want)


def tiny_qwen3(layers=1):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=layers,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=4096)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    return Qwen3ForCausalLM(cfg).eval()


def test_session_plumbing_on_host():
    from prismkv_amd.hf import HFNative
    model = tiny_qwen3()
    with pytest.raises(ValueError, match="missing"):
        HFNative(model, {})
    with pytest.raises(NotImplementedError, match="16 buckets"):
        HFNative(model, encoders(1), selected_buckets=8)
    with pytest.raises(ValueError, match="unique cap"):
        HFNative(model, encoders(1), unique_cap=1.5)
    ids = torch.randint(0, 128, (1, 12))
    with torch.no_grad():
        dense = model(ids).logits
    session = HFNative(model, encoders(1))
    assert model.config._attn_implementation == "prismkv_native"
    with torch.no_grad():
        prefill = model(ids).logits  # prefill runs the model's own SDPA attention
    assert torch.equal(prefill, dense)
    assert session.prefix_lengths == {0: 12}
    with pytest.raises(ValueError, match="already has"):
        HFNative(model, encoders(1))
    session.close()
    assert model.config._attn_implementation == "sdpa"


def test_static_cache_session_on_host():
    from transformers import StaticCache
    from prismkv_amd.hf import DecodeGraph, HFNative
    model = tiny_qwen3()
    ids = torch.randint(0, 128, (1, 12))
    with torch.no_grad():
        dense = model(ids).logits[:, -1]
    session = HFNative(model, encoders(1), router="q_activation")
    with pytest.raises(NotImplementedError, match="moments router"):
        DecodeGraph(session, StaticCache(config=model.config, max_cache_len=32))
    session.close()
    session = HFNative(model, encoders(1))
    cache = StaticCache(config=model.config, max_cache_len=32)
    step = DecodeGraph(session, cache)
    with pytest.raises(ValueError, match="already drives"):
        DecodeGraph(session, cache)
    with pytest.raises(RuntimeError, match="prefill every layer"):
        step(ids[:, :1])
    # the prefill over the static buffers (explicit causal mask from the
    # positions) gives the dense model's logits
    with torch.no_grad(), session.prefill():
        static = model(ids, position_ids=torch.arange(12)[None], past_key_values=cache, use_cache=True).logits[:, -1]
    assert torch.allclose(static, dense, atol=1e-5, rtol=1e-5)
    assert session.prefix_lengths == {0: 12} and session._capacity(13) == 32
    step.close()
    assert session._static is None
    session.close()


def test_detailed_record_fields_from_bitmaps():
    # the detailed record fields (src/prismkv/hf_reference.py:216-231) computed
    # from the device layout -- ascending ids with a count, bitmap rows of the
    # kept buckets -- equal a direct count over the bucket lists
    from types import SimpleNamespace
    from prismkv_amd.hf import _old_unique_raw, _popcount32
    words = torch.tensor([0, 1, -1, 0x7FFFFFFF, -2147483648, 0x55555555], dtype=torch.int32)
    assert _popcount32(words).tolist() == [0, 1, 32, 31, 1, 16]
    gen = torch.Generator().manual_seed(9)
    H, width, row_words = 300, 16, 12
    lists = [[torch.unique(torch.randint(0, H, (int(torch.randint(0, 40, (1,), generator=gen)),), generator=gen))
              for _ in range(3000)] for _ in range(8)]
    bits = torch.zeros(8, 3000, row_words, dtype=torch.int64)
    for g in range(8):
        for f in range(3000):
            for t in lists[g][f].tolist():
                bits[g, f, t // 32] |= 1 << (t % 32)
    bits = torch.where(bits >= 2 ** 31, bits - 2 ** 32, bits).to(torch.int32)
    features = torch.randint(0, 3000, (8, width), generator=gen)
    valid = (torch.rand(8, width, generator=gen) > 0.3).float()
    ids = torch.zeros(8, H, dtype=torch.int32)
    count = torch.zeros(8, dtype=torch.int32)
    for g in range(8):
        u = torch.unique(torch.cat([lists[g][int(f)] for f, ok in zip(features[g], valid[g]) if ok > 0] +
                                   [torch.zeros(0, dtype=torch.long)]))
        ids[g, :len(u)] = u.int()
        count[g] = len(u)
    op = SimpleNamespace(ids=ids, count=count, bits=bits, features=features, valid=valid)
    for prefix in (0, 1, 31, 32, 33, 100, 299, 300):
        old_unique, old_raw = _old_unique_raw(op, prefix)
        for g in range(8):
            kept = [int(f) for f, ok in zip(features[g], valid[g]) if ok > 0]
            assert int(old_unique[g]) == int((ids[g, :count[g]] < prefix).sum())
            assert int(old_raw[g]) == sum(int((lists[g][f] < prefix).sum()) for f in kept), (prefix, g)
