"""The trained-encoder fixture (`qwen3_8b_encoders.npz`, written by
`make_trained_encoders.py` from the reference's pretrained/Qwen3-8B bundle)
and the inputs the tests build around it.

The fixture holds 4 of the bundle's 288 units.  A layer of 8 KV groups uses
unit g mod 4 for group g, so every unit serves two groups with different
keys.  Keys are synthetic (the backbone is not available): per group, a
16-component Gaussian mixture in the encoder's normalised space, scaled by
the unit's saved key scale and shifted by a per-group offset, so that the
center and the scale the build applies matter and bucket sizes are skewed.
"""
from pathlib import Path

import numpy as np

FIXTURE = Path(__file__).with_name("qwen3_8b_encoders.npz")
UNITS = 4


def load():
    with np.load(FIXTURE, allow_pickle=False) as f:
        return {name: f[name] for name in f.files}


def group_tables(fx, groups=8):
    """Per-group encoder tables of one layer: W f32 [G,3000,128], b f32
    [G,3000], key and query scales f32 [G] (the fp32 values the device
    divides by), and the unit index of each group."""
    units = np.arange(groups) % len(fx["layer"])
    return (np.ascontiguousarray(fx["W_enc"][units]), np.ascontiguousarray(fx["b_enc"][units]),
            fx["key_scale"][units].astype(np.float32), fx["query_scale"][units].astype(np.float32), units)


def mixture_keys(rows, key_scale, seed, device="cuda"):
    """bf16 keys [G, rows, 128]: 16-component mixture (centers N(0, 0.8^2),
    spread 0.6) times the group's key scale, plus a N(0, 0.5^2) offset."""
    import torch
    G = len(key_scale)
    gen = torch.Generator(device=device).manual_seed(seed)
    centers = torch.randn(G, 16, 128, generator=gen, device=device) * 0.8
    comp = torch.randint(0, 16, (G, rows), generator=gen, device=device)
    x = torch.gather(centers, 1, comp[..., None].expand(-1, -1, 128))
    x += 0.6 * torch.randn(G, rows, 128, generator=gen, device=device)
    offset = torch.randn(G, 1, 128, generator=gen, device=device) * 0.5
    scale = torch.as_tensor(np.asarray(key_scale, np.float32), device=device)[:, None, None]
    return (x * scale + offset).to(torch.bfloat16)
