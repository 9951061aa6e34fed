"""Encoder bundles: the SAE encoders and Q/K scales of every (layer, KV
group), in the reference's on-disk format (src/prismkv/weights.py:18-70):
one tensor-only file `l{layer:02d}_g{group:02d}.pt` holding W_enc f32
[3000,128] and b_enc f32 [3000] per group, plus `manifest.json` (schema 1)
with each file's sha256, shapes, key_mean, query_topk and the saved
key/query scales.

`SharedSAE` is the encoder half of the reference module
(src/prismkv/core.py:29-48): same parameter names, shapes and initialisation
(W_enc kaiming-uniform, b_enc zero, W_dec = W_enc^T), `dense` = relu(x W^T + b)
in fp32.  Loading never unpickles code (`torch.load(weights_only=True)`).
`layer_tables` stacks one layer's 8 groups into the device tables that
`Native8B.from_keys` / `set_encoder_tables` take.
"""
from __future__ import annotations

import hashlib
import json
import math
from dataclasses import dataclass
from pathlib import Path

import torch
from torch import nn
from torch.nn import functional as F


class SharedSAE(nn.Module):
    """Encoder of one (layer, KV group) -- src/prismkv/core.py:29-48."""

    def __init__(self, head_dim=128, features=3000, key_mean=8, query_topk=16):
        super().__init__()
        if not 1 <= key_mean <= features or not 1 <= query_topk <= features:
            raise ValueError("invalid sparsity")
        self.head_dim, self.features = head_dim, features
        self.key_mean, self.query_topk = key_mean, query_topk
        self.W_enc = nn.Parameter(torch.empty(features, head_dim))
        nn.init.kaiming_uniform_(self.W_enc, a=math.sqrt(5))
        self.b_enc = nn.Parameter(torch.zeros(features))
        self.W_dec = nn.Parameter(self.W_enc.detach().T.clone())
        self.b_dec = nn.Parameter(torch.zeros(head_dim))
        self.register_buffer("seen", torch.tensor(0))
        self.register_buffer("last", torch.zeros(features, dtype=torch.long))
        self.register_buffer("counts", torch.zeros(features, dtype=torch.long))

    def dense(self, normalized):
        return F.linear(normalized.float(), self.W_enc.float(), self.b_enc.float()).relu()


@dataclass
class Encoder:
    """src/prismkv/hf_reference.py:16-20."""

    sae: object
    key_scale: float
    query_scale: float


def _sha(path):
    digest = hashlib.sha256()
    with Path(path).open("rb") as fh:
        while block := fh.read(8 << 20):
            digest.update(block)
    return digest.hexdigest()


MANIFEST = "manifest.json"
FORMAT = "PrismKV inference encoder bundle; decoder/optimizer omitted"


def _unit_file(layer, group):
    return f"l{layer:02d}_g{group:02d}.pt"


def save_encoders(encoders, directory, *, metadata=None):
    """Write one tensor-only file per (layer, group) and the manifest into a
    new directory (src/prismkv/weights.py:18-38: the same names and fields)."""
    root = Path(directory)
    root.mkdir(parents=True, exist_ok=False)  # never overwrite a bundle
    rows = []
    for unit in sorted(encoders):
        layer, group = unit
        enc = encoders[unit]
        if min(layer, group) < 0 or not (enc.key_scale > 0 and enc.query_scale > 0):
            raise ValueError("invalid group or saved scale")
        sae, name = enc.sae, _unit_file(layer, group)
        torch.save({"W_enc": sae.W_enc.detach().float().cpu(), "b_enc": sae.b_enc.detach().float().cpu()},
                   root / name)
        rows.append({"layer": layer, "group": group, "file": name, "sha256": _sha(root / name),
                     "head_dim": sae.head_dim, "features": sae.features, "key_mean": sae.key_mean,
                     "query_topk": sae.query_topk, "key_scale": float(enc.key_scale),
                     "query_scale": float(enc.query_scale)})
    text = json.dumps({"schema": 1, "format": FORMAT, "metadata": metadata or {}, "groups": rows}, indent=2)
    (root / MANIFEST).write_text(text, encoding="utf8")


def _checked_tensors(root, row):
    """The row's file, verified to sit in the bundle and to match its hash,
    loaded without unpickling code."""
    path = (root / row["file"]).resolve()
    if path.parent != root or _sha(path) != row["sha256"]:
        raise ValueError("encoder path/hash mismatch")
    tensors = torch.load(path, map_location="cpu", weights_only=True)
    if set(tensors) != {"W_enc", "b_enc"}:
        raise ValueError("unexpected checkpoint contents")
    return tensors


def _encoder_from_row(row, tensors, device):
    with torch.random.fork_rng(devices=[]):  # loading leaves the caller's RNG stream alone
        sae = SharedSAE(row["head_dim"], row["features"], row["key_mean"], row["query_topk"])
    for name in ("W_enc", "b_enc"):
        if tensors[name].shape != getattr(sae, name).shape:
            raise ValueError("encoder shape mismatch")
    if not all(bool(torch.isfinite(t).all()) for t in tensors.values()):
        raise ValueError("nonfinite encoder")
    with torch.no_grad():
        sae.W_enc.copy_(tensors["W_enc"])
        sae.b_enc.copy_(tensors["b_enc"])
    sae.to(device).eval().requires_grad_(False)
    if not (row["key_scale"] > 0 and row["query_scale"] > 0):
        raise ValueError("positive Q/K scales required")
    return Encoder(sae, row["key_scale"], row["query_scale"])


def load_encoders(directory, *, device="cpu"):
    """-> ({(layer, group): Encoder}, manifest), with the reference's checks
    and error messages (src/prismkv/weights.py:41-70): schema, file inside
    the bundle, sha256, tensor names, shapes, finiteness, positive scales,
    no duplicate unit."""
    root = Path(directory).resolve()
    manifest = json.loads((root / MANIFEST).read_text(encoding="utf8"))
    if manifest.get("schema") != 1:
        raise ValueError("unsupported encoder-bundle schema")
    out = {}
    for row in manifest["groups"]:
        tensors = _checked_tensors(root, row)
        unit = (row["layer"], row["group"])
        if unit in out:
            raise ValueError("duplicate layer/KV group")
        out[unit] = _encoder_from_row(row, tensors, device)
    return out, manifest


def layer_tables(encoders, layer, groups=8, device=None):
    """One layer's encoders as device tables: W [groups,3000,128] f32,
    b [groups,3000] f32, key_scale [groups] f32 and the shared key_mean."""
    units = [encoders[(layer, g)] for g in range(groups)]
    means = {int(u.sae.key_mean) for u in units}
    if len(means) != 1:
        raise ValueError("all groups of a layer must share one key_mean")
    W = torch.stack([u.sae.W_enc.detach().float() for u in units]).to(device)
    b = torch.stack([u.sae.b_enc.detach().float() for u in units]).to(device)
    scale = torch.tensor([float(u.key_scale) for u in units], dtype=torch.float32, device=device)
    return W.contiguous(), b.contiguous(), scale, means.pop()
