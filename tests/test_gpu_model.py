"""The 36-layer decode step at the Qwen3-8B attention geometry, end to end
through the native Hugging Face backend: a random-init bf16 Qwen3 with 36
layers, 32 query / 8 KV heads, head_dim 128, hidden 4096, MLP 12288 (vocab
reduced to 32000), 32768 prefilled synthetic tokens, then 512 generated
tokens decoded one by one (each layer's index is built on the device at the
first decode step; the 512-token tail is attended densely).  At the last
step:
  * every third layer (and the last) is checked in full against the oracle's
    route + attention (src/prismkv/core.py:106-183) over the index the device
    holds, and every layer reports no device error;
  * every layer's Top-16 sparse output is compared with the all-read dense
    attention over the same 33280 rows (exact fp32 softmax on the device):
    the per-layer deviation of sparse from dense that the configuration
    names, logged for all 36 layers (a measure of the routing's
    approximation on this random-weight model, not a parity bar).
"""
import numpy as np
import pytest
import torch

from tests.gpu_util import log
from tests.test_gpu_hf import Capture, check_call

pytestmark = pytest.mark.gpu


def dense_deviation(q, K, V, out):
    """Relative L2 of the sparse output from the exact all-read attention of
    the same 4 heads per group over every row (fp32 on the device)."""
    qf = q.float()                                   # [8, 4, 128]
    kt = K.float().transpose(1, 2).contiguous()      # [8, 128, rows]
    p = torch.softmax((qf @ kt) / 128 ** 0.5, dim=-1)
    dense = p @ V.float()                            # [8, 4, 128]
    sparse = out.float()
    return float((sparse - dense).norm() / dense.norm())


def test_qwen3_8b_geometry_36_layer_step():
    from transformers import DynamicCache, Qwen3Config, Qwen3ForCausalLM
    from prismkv_amd.hf import HFNative
    from prismkv_amd.weights import Encoder, SharedSAE
    L, P, T = 36, 32768, 512
    cfg = Qwen3Config(vocab_size=32000, hidden_size=4096, intermediate_size=12288, num_hidden_layers=L,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=40960)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    previous = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("cuda"):
            model = Qwen3ForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(previous)
    gen = torch.Generator().manual_seed(21)
    encoders = {}
    for layer in range(L):
        for g in range(8):
            sae = SharedSAE()
            with torch.no_grad():
                sae.W_enc.copy_(torch.randn(3000, 128, generator=gen) / 128 ** 0.5)
            encoders[(layer, g)] = Encoder(sae, 1.0, 1.0)
    session = HFNative(model, encoders)
    ids = torch.randint(0, 32000, (1, P + T), generator=torch.Generator().manual_seed(22)).cuda()
    cache = DynamicCache(config=cfg)
    with torch.no_grad():
        for lo in range(0, P, 8192):  # chunked prefill through the model's own attention
            with session.prefill():
                model(ids[:, lo:lo + 8192], past_key_values=cache, use_cache=True, logits_to_keep=1)
        for s in range(T - 1):
            model(ids[:, P + s:P + s + 1], past_key_values=cache, use_cache=True, logits_to_keep=1)
        torch.cuda.synchronize()
        log(f"prefill {P} + {T - 1} decode steps done")
        cap = Capture(session)
        model(ids[:, P + T - 1:P + T], past_key_values=cache, use_cache=True, logits_to_keep=1)
        torch.cuda.synchronize()
    assert len(cap.calls) == L
    for layer, op in session.ops.items():
        assert op.history == P and op.decode_errors() == 0, layer
    checked = set(range(0, L, 3)) | {L - 1}
    deviation = {}
    for layer, q, K, V, out in cap.calls:
        assert K.shape[1] == P + T
        if layer in checked:
            err = check_call(session.ops[layer], layer, q, K, V, out)
            log(f"  layer {layer}: history={P} tail={T} {err}")
        deviation[layer] = dense_deviation(q, K, V, out)
    log("  sparse vs all-read dense attention, relative L2 per layer: " +
        " ".join(f"{layer}:{deviation[layer]:.3f}" for layer in sorted(deviation)))
    dev = np.array([deviation[layer] for layer in sorted(deviation)])
    log(f"  deviation over the 36 layers: mean {dev.mean():.3f}, min {dev.min():.3f}, max {dev.max():.3f}")
    assert len(dev) == L and np.isfinite(dev).all()
    recs = session.records[-L * 8:]
    assert all(r["tail"] == T and r["buckets"] == 16 for r in recs)
    log(f"  unique ids per group, last step: mean {np.mean([r['unique'] for r in recs]):.0f}")
    session.close()
