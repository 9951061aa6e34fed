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
