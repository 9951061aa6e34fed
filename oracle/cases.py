"""Seeded input cases for the parity tests -- TEST INFRASTRUCTURE ONLY.

* `native_case` restates the six synthetic witnesses of
  examples/check_native8b.py:14-31,80 (membership constructions "ties",
  "few", "random", "empty"; moments of the original keys; zeroed moments for
  "ties") with numpy's seeded PCG64 generator instead of the device RNG.
* `replay_case` is the CPU replay shape (examples/replay.py): H=1024, T=32,
  keys/queries N(0,1), SAE W_enc ~ N(0, 1/128), b = 0, index built with the
  reference's global BatchTopK budget 8*H (src/prismkv/core.py:92-103).
* `topk8_case` is the 8B-geometry kernel check: bf16 K/V ~ N(0,1), every key
  joins the buckets of its top-8 ReLU activations of the same random SAE.
* `update_case` is one append_index step (src/prismkv/core.py:186-201): an
  index built by the reference rule over the first H keys, then a block of N
  new keys to index with the same per-group SAE and key scale.  Its kinds
  steer the BatchTopK branches of src/prismkv/core.py:13-26: "random"
  (distinct values), "bias_ties" (W = 0, b = 1: every activation equals 1,
  so ties at tau overflow the budget and the flat-index order decides),
  "sparse" (b = -3: fewer positives than the budget, tau = 0), "dead"
  (b = -100: no positive activation at all) and "dup" (the block's keys
  come in identical pairs: ties of two at every value).
* `build_case` is one prefill index build (src/prismkv/core.py:92-103) of
  the first H keys of each group with the SAEs and kinds of `update_case`,
  plus V, Q and a T-row tail for a decode step on the built index.

All cases return plain numpy arrays: bf16 tensors as uint16 bit patterns,
indices as `oracle.Index` objects.
"""
from __future__ import annotations

import numpy as np

from . import Index, bf16_to_f32, build_index, f32_to_bf16, summarize

G, HQ, D, F, TOPK = 8, 4, 128, 3000, 16

# examples/check_native8b.py:80
NATIVE_CASES = [(32, 1, "ties"), (65, 7, "few"), (257, 31, "random"), (257, 129, "empty"), (1025, 3, "random"),
                (65536, 17, "random")]
# memberships per group reported by reviewer_guide/native8b_validation.json for those cases
NATIVE_MEMBERSHIPS = {(32, "ties"): 32, (65, "few"): 65, (257, "random"): 771, (257, "empty"): 0,
                      (1025, "random"): 3075, (65536, "random"): 196608}


def normal(seed, shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(scale))


def bf16_normal(seed, shape):
    return f32_to_bf16(normal(seed, shape))


def native_lists(H, kind, g):
    """Per-bucket ascending token lists of examples/check_native8b.py:14-21."""
    if kind == "empty":
        tid = np.empty(0, np.int64)
        fid = np.empty(0, np.int64)
    elif kind == "ties":
        tid = np.arange(H, dtype=np.int64)
        fid = tid % min(H, 64)
    elif kind == "few":
        tid = np.arange(H, dtype=np.int64)
        fid = (tid + g) % 7
    elif kind == "random":
        tid = np.repeat(np.arange(H, dtype=np.int64), 3)
        fid = np.stack([(np.arange(H) + g * 17 + off) % F for off in (0, 137, 811)], axis=-1).reshape(-1)
    else:
        raise ValueError(kind)
    order = np.argsort(fid, kind="stable")
    counts = np.bincount(fid, minlength=F)
    bounds = np.concatenate(([0], np.cumsum(counts)))
    tid_sorted = tid[order]
    return [tid_sorted[bounds[f]:bounds[f + 1]] for f in range(F)]


def index_from_lists(keys_f32, lists, zero_moments=False):
    counts, mean, var = summarize(keys_f32, lists)
    if zero_moments:
        mean[:] = 0
        var[:] = 0
    return Index(len(keys_f32), keys_f32.mean(0), counts, mean, var, lists)


def native_case(H, tail, kind, seed=None):
    """Inputs of one examples/check_native8b.py case (8 groups)."""
    seed = 90 + H if seed is None else seed
    k = bf16_normal((seed, 0), (G, H + tail, D))
    v = bf16_normal((seed, 1), (G, H + tail, D))
    q = bf16_normal((seed, 2), (G, HQ, D))
    kf = bf16_to_f32(k)
    indices = [index_from_lists(kf[g, :H], native_lists(H, kind, g), zero_moments=(kind == "ties"))
               for g in range(G)]
    return dict(H=H, T=tail, q=q, k=k, v=v, indices=indices, kind=kind)


def sae_weights(seed, g=0, features=F, dim=D):
    """Random SAE encoder W_enc ~ N(0, 1/dim), b = 0."""
    return normal((seed, 100 + g), (features, dim), scale=1.0 / np.sqrt(dim)), np.zeros(features, np.float32)


def replay_case(seed=5, H=1024, T=32, bf16=True):
    """CPU replay shape with the reference global-budget index per group."""
    k32 = normal((seed, 0), (G, H + T, D))
    v32 = normal((seed, 1), (G, H + T, D))
    q32 = normal((seed, 2), (G, HQ, D))
    if bf16:
        k, v, q = f32_to_bf16(k32), f32_to_bf16(v32), f32_to_bf16(q32)
        kf = bf16_to_f32(k)
    else:
        k, v, q, kf = k32, v32, q32, k32
    indices = []
    for g in range(G):
        W, b = sae_weights(seed, g)
        indices.append(build_index(kf[g, :H], W, b, 1.0, key_mean=8))
    return dict(H=H, T=T, q=q, k=k, v=v, indices=indices, kind="replay")


def topk8_lists(keys_f32, W, b, per_key=8, block=8192):
    """Every key joins the buckets of its top-`per_key` positive ReLU activations."""
    H = len(keys_f32)
    toks, feats = [], []
    for lo in range(0, H, block):
        a = keys_f32[lo:lo + block] @ W.T + b
        top = np.argpartition(-a, per_key - 1, axis=1)[:, :per_key]
        val = np.take_along_axis(a, top, 1)
        rows = np.repeat(np.arange(lo, lo + len(a)), per_key).reshape(len(a), per_key)
        keep = val > 0
        toks.append(rows[keep])
        feats.append(top[keep])
    tid = np.concatenate(toks).astype(np.int64)
    fid = np.concatenate(feats).astype(np.int64)
    order = np.lexsort((tid, fid))
    counts = np.bincount(fid, minlength=W.shape[0])
    bounds = np.concatenate(([0], np.cumsum(counts)))
    tid = tid[order]
    return [tid[bounds[f]:bounds[f + 1]] for f in range(W.shape[0])]


def topk8_case(H=65536, T=256, seed=2, groups=G):
    """8B-geometry kernel check inputs (per-key top-8 membership)."""
    k = bf16_normal((seed, 0), (groups, H + T, D))
    v = bf16_normal((seed, 1), (groups, H + T, D))
    q = bf16_normal((seed, 2), (groups, HQ, D))
    kf = bf16_to_f32(k)
    indices = []
    for g in range(groups):
        W, b = sae_weights(seed, g)
        indices.append(index_from_lists(kf[g, :H], topk8_lists(kf[g, :H], W, b)))
    return dict(H=H, T=T, q=q, k=k, v=v, indices=indices, kind="topk8")


UPDATE_KINDS = ("random", "bias_ties", "sparse", "dead", "dup")


def update_sae(kind, seed, g):
    W, b = sae_weights(seed, g)
    if kind == "bias_ties":
        W = np.zeros_like(W)
        b = np.ones_like(b)
    elif kind == "sparse":
        b = np.full_like(b, -3.0)
    elif kind == "dead":
        b = np.full_like(b, -100.0)
    return W, b


def update_case(kind="random", H=512, N=256, T=8, seed=21, key_mean=8):
    """Inputs of one append step for 8 groups (see the module docstring)."""
    k = bf16_normal((seed, 0), (G, H + N + T, D))
    if kind == "dup":
        k[:, H + 1:H + N:2] = k[:, H:H + N - 1:2]
    v = bf16_normal((seed, 1), (G, H + N + T, D))
    q = bf16_normal((seed, 2), (G, HQ, D))
    kf = bf16_to_f32(k)
    W = np.empty((G, F, D), np.float32)
    b = np.empty((G, F), np.float32)
    scale = np.array([1.0 + 0.25 * g for g in range(G)], np.float32)
    indices = []
    for g in range(G):
        W[g], b[g] = update_sae(kind, seed, g)
        indices.append(build_index(kf[g, :H], W[g], b[g], float(scale[g]), key_mean=key_mean))
    return dict(H=H, N=N, T=T, q=q, k=k, v=v, W=W, b=b, scale=scale, key_mean=key_mean, indices=indices, kind=kind)


def build_case(kind="random", H=1024, T=8, seed=51, key_mean=8):
    """Inputs of one prefill index build for 8 groups (see the module docstring)."""
    k = bf16_normal((seed, 0), (G, H + T, D))
    if kind == "dup":
        k[:, 1:H:2] = k[:, 0:H - 1:2]
    v = bf16_normal((seed, 1), (G, H + T, D))
    q = bf16_normal((seed, 2), (G, HQ, D))
    W = np.empty((G, F, D), np.float32)
    b = np.empty((G, F), np.float32)
    for g in range(G):
        W[g], b[g] = update_sae(kind, seed, g)
    scale = np.array([1.0 + 0.25 * g for g in range(G)], np.float32)
    return dict(H=H, T=T, q=q, k=k, v=v, W=W, b=b, scale=scale, key_mean=key_mean, kind=kind)
