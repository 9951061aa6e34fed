"""Helpers shared by the GPU parity tests: move an oracle case to the device
and build the MI355X operator from it."""
import sys

import numpy as np
import torch

from prismkv_amd import FeatureIndex, Native8B


def log(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def bf16_tensor(bits, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def bf16_bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def device_indices(case, device="cuda"):
    out = []
    for i in case["indices"]:
        out.append(FeatureIndex(i.history, torch.from_numpy(i.center).to(device),
                                torch.from_numpy(i.counts).to(device), torch.from_numpy(i.mean).to(device),
                                torch.from_numpy(i.variance).to(device), [torch.from_numpy(l) for l in i.lists]))
    return out


def operator(case, **kwargs):
    op = Native8B(device_indices(case), **kwargs)
    return op, bf16_tensor(case["q"]), bf16_tensor(case["k"]), bf16_tensor(case["v"])


def route_outputs(op):
    torch.cuda.synchronize()
    return (op.features.cpu().numpy(), op.valid.cpu().numpy(), op.raw.cpu().numpy(), op.ids.cpu().numpy(),
            op.count.cpu().numpy())


def device_layer(H, T, seed, device="cuda"):
    """A layer built on the device for histories too long for the oracle's
    case generator: bf16 K/V/Q ~ N(0,1) and, per group, each key in the
    buckets of its positive top-8 activations of a random SAE; moments from
    those members.  Returns (op, q, k, v)."""
    G, HQ, D, F = 8, 4, 128, 3000
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    k = torch.randn(G, H + T, D, generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn(G, H + T, D, generator=gen, device=device).to(torch.bfloat16)
    q = torch.randn(G, HQ, D, generator=gen, device=device).to(torch.bfloat16)
    counts = torch.zeros(G, F, dtype=torch.int64, device=device)
    mean = torch.zeros(G, F, D, device=device)
    var = torch.zeros(G, F, D, device=device)
    csr, offs = [], []
    for g in range(G):
        W = torch.randn(F, D, generator=gen, device=device) / D ** 0.5
        keys = k[g, :H].float()
        toks, feats = [], []
        for lo in range(0, H, 16384):
            val, idx = (keys[lo:lo + 16384] @ W.T).topk(8, dim=1)
            keep = val > 0
            toks.append(torch.arange(lo, lo + len(val), device=device)[:, None].expand_as(idx)[keep])
            feats.append(idx[keep])
        tok, feat = torch.cat(toks), torch.cat(feats)
        order = torch.argsort(feat * H + tok)
        tok, feat = tok[order], feat[order]
        n = torch.bincount(feat, minlength=F)
        counts[g] = n
        mu = torch.zeros(F, D, device=device).index_add_(0, feat, keys[tok]) / n.clamp_min(1)[:, None]
        dev = keys[tok] - mu[feat]
        mean[g] = mu
        var[g] = torch.zeros(F, D, device=device).index_add_(0, feat, dev * dev) / n.clamp_min(1)[:, None]
        csr.append(tok.int())
        offs.append(torch.cat((torch.zeros(1, dtype=torch.int64, device=device), n.cumsum(0))).int())
    width = max(len(x) for x in csr)
    csr = torch.stack([torch.nn.functional.pad(x, (0, width - len(x))) for x in csr])
    op = Native8B.from_tables(H, counts, mean, var, csr, torch.stack(offs))
    return op, q, k, v
