"""The trained-encoder fixture and the reference's Qwen3-8B bundle on the CPU
(no GPU needed):

  * the fixture's 4 units have the bundle's shapes, sparsity settings and
    positive scales (pretrained/README.md:9-13);
  * where the reference bundle is present (pretrained/Qwen3-8B, 288 units),
    `load_encoders` reads all of it with its sha256 and tensor checks
    (src/prismkv/weights.py:41-70), every layer stacks into device tables,
    and the fixture's units equal the bundle's bit for bit;
  * on trained tables the C oracle's append_index and the torch-CPU
    restatement (the same torch operations as src/prismkv/core.py:92-103,
    :186-201) agree: memberships identical or different only within the
    encode rounding of the threshold, counts and moments within fp32
    rounding.  The mixed-sign bias of trained encoders puts about half of
    the activations at zero and moves the threshold, which random SAEs with
    b = 0 never do.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from oracle import expect, torch_cpu
from tests.golden import trained

BUNDLE = Path("/root/reference/pretrained/Qwen3-8B")


def test_fixture_shapes_and_scales():
    fx = trained.load()
    n = len(fx["layer"])
    assert n == trained.UNITS
    assert fx["W_enc"].shape == (n, 3000, 128) and fx["W_enc"].dtype == np.float32
    assert fx["b_enc"].shape == (n, 3000) and fx["b_enc"].dtype == np.float32
    assert np.isfinite(fx["W_enc"]).all() and np.isfinite(fx["b_enc"]).all()
    assert (fx["key_scale"] > 0).all() and (fx["query_scale"] > 0).all()
    assert (fx["key_mean"] == 8).all() and (fx["query_topk"] == 16).all()
    # the trained biases are of mixed sign (a random SAE's are zero)
    assert ((fx["b_enc"] < 0).sum(1) > 1000).all() and ((fx["b_enc"] > 0).sum(1) > 1000).all()
    for i in range(n):
        assert fx["unit_file"][i] == f"l{fx['layer'][i]:02d}_g{fx['group'][i]:02d}.pt"


@pytest.mark.skipif(not BUNDLE.is_dir(), reason="the reference's encoder bundle is not present")
def test_reference_bundle_loads_and_matches_the_fixture():
    from prismkv_amd.weights import layer_tables, load_encoders
    encoders, manifest = load_encoders(BUNDLE)
    assert manifest["schema"] == 1 and len(encoders) == 288
    assert sorted(encoders) == [(l, g) for l in range(36) for g in range(8)]
    for layer in range(36):
        W, b, scale, key_mean = layer_tables(encoders, layer)
        assert W.shape == (8, 3000, 128) and b.shape == (8, 3000) and scale.shape == (8,) and key_mean == 8
        assert bool((scale > 0).all())
    rows = {(r["layer"], r["group"]): r for r in manifest["groups"]}
    fx = trained.load()
    for i in range(len(fx["layer"])):
        unit = (int(fx["layer"][i]), int(fx["group"][i]))
        enc = encoders[unit]
        assert np.array_equal(enc.sae.W_enc.detach().numpy(), fx["W_enc"][i]), unit
        assert np.array_equal(enc.sae.b_enc.detach().numpy(), fx["b_enc"][i]), unit
        assert enc.key_scale == fx["key_scale"][i] and enc.query_scale == fx["query_scale"][i], unit
        assert rows[unit]["sha256"] == fx["sha256"][i] and rows[unit]["file"] == fx["unit_file"][i], unit


@pytest.mark.parametrize("unit", range(trained.UNITS))
def test_oracles_agree_on_trained_tables(unit):
    fx = trained.load()
    W, b = fx["W_enc"][unit], fx["b_enc"][unit]
    scale = np.float32(fx["key_scale"][unit])
    rng = np.random.default_rng(400 + unit)
    H, N = 384, 160
    # mixture keys around an offset, scaled by the unit's key scale
    centers = rng.standard_normal((16, 128)).astype(np.float32) * 0.8
    x = centers[rng.integers(0, 16, H + N)] + 0.6 * rng.standard_normal((H + N, 128)).astype(np.float32)
    keys = (x * scale + 0.5 * rng.standard_normal(128).astype(np.float32)).astype(np.float32)
    idx0 = oracle.build_index(keys[:H], W, b, scale, 8)
    c_idx, act = oracle.append_index(idx0, keys[H:], W, b, scale, 8, return_act=True)
    counts, mean, var, lists = torch_cpu.append_block(
        torch.from_numpy(idx0.counts), torch.from_numpy(idx0.mean), torch.from_numpy(idx0.variance),
        [torch.from_numpy(l) for l in idx0.lists], H, torch.from_numpy(idx0.center), torch.from_numpy(keys[H:]),
        torch.from_numpy(W), torch.from_numpy(b), float(scale))
    xb = (keys[H:] - idx0.center) / scale
    bound = expect.encode_error_bound(xb, W, b)
    block = lambda ls: [np.asarray(l)[np.asarray(l) >= H] - H for l in ls]  # noqa: E731
    moved = expect.check_memberships(block(c_idx.lists), block([l.numpy() for l in lists]), act, 8 * N, bound,
                                     f"unit {unit}")
    zero = float((act == 0).mean())
    assert zero > 0.3  # the negative biases silence a large share of the activations
    if moved == 0:
        assert np.array_equal(counts.numpy(), c_idx.counts)
        assert np.allclose(mean.numpy(), c_idx.mean, rtol=1e-5, atol=1e-5 * float(scale))
        assert np.allclose(var.numpy(), c_idx.variance, rtol=1e-4, atol=1e-5 * float(scale) ** 2)
    print(f"unit {unit}: zero activations {zero:.2f}, memberships moved at tau {moved}")
