"""Torch-CPU restatement of the reference's per-group decode step and index
update -- TEST AND BASELINE INFRASTRUCTURE ONLY.

bench.py's `cpu_baseline` leg times these functions on the host cores (the
reference's own CPU path cannot travel to the GPU box), and
tests/test_oracle_torch.py pins them against the C oracle.  They use the
same torch CPU operations, dtypes and per-bucket Python loops as the
reference, so that the timing is that of the reference's CPU path:

* moment_route        src/prismkv/core.py:106-130 (router "moments")
* union_walk          src/prismkv/core.py:142-167 (per-bucket mask walk, optional strict cap)
* attend_rows         src/prismkv/core.py:170-183
* append_block        src/prismkv/core.py:13-26, :47-48, :76-103, :186-201

Nothing here is imported by the package; the product path never runs it.
"""
from __future__ import annotations

import math

import torch


def moment_route(q, counts, mean, var, topk=16):
    """Shared bucket scores of one group's query heads and the ranked live
    buckets (at most `topk`): logit = (log max(n, 1) + q.mean / sqrt(d)) +
    q^2.var / (2 d), dead buckets -inf, softmax over buckets per head, mean
    over heads, stable descending order (core.py:118-130)."""
    qf = q.float()
    d = qf.shape[-1]
    alive = counts > 0
    if not bool(alive.any()):
        return torch.zeros(counts.shape[0]), torch.zeros(0, dtype=torch.long)
    logits = counts.clamp_min(1).float().log().expand(qf.shape[0], -1).clone()
    logits += (qf @ mean.T) / math.sqrt(d)
    logits += (qf * qf) @ var.T / (2 * d)
    logits[:, ~alive] = float("-inf")
    score = torch.softmax(logits, dim=-1).mean(dim=0)
    ranked = torch.argsort(score, descending=True, stable=True)
    return score, ranked[alive[ranked]][:topk]


def union_walk(order, lists, history, unique_cap=None):
    """Walk the ranked buckets over a boolean token mask, skipping a bucket
    whose new tokens would overflow floor(history * unique_cap) (core.py:149-
    163); returns (ascending token ids, kept buckets, raw)."""
    limit = history if unique_cap is None else math.floor(history * unique_cap)
    taken = torch.zeros(history, dtype=torch.bool)
    kept, raw, unique = [], 0, 0
    for b in order.tolist():
        members = lists[b]
        fresh = int((~taken[members]).sum())
        if unique + fresh <= limit:
            taken[members] = True
            unique += fresh
            raw += len(members)
            kept.append(b)
    return taken.nonzero().flatten(), kept, raw


def attend_rows(q, keys, values, ids, history):
    """Exact fp32 softmax attention over rows `ids` (< history) and the tail
    [history, len(keys)), scale 1/sqrt(d), cast back to q's dtype
    (core.py:170-183)."""
    rows = torch.cat((ids, torch.arange(history, keys.shape[0])))
    if rows.numel() == 0:
        return torch.zeros_like(q)
    logits = (q.float() @ keys[rows].float().T) / math.sqrt(q.shape[-1])
    return (torch.softmax(logits, dim=-1) @ values[rows].float()).to(q.dtype)


def decode_group(q, counts, mean, var, lists, keys, values, history, unique_cap=None):
    """One group's decode step: route, union walk, attention."""
    _, order = moment_route(q, counts, mean, var)
    ids, _, _ = union_walk(order, lists, history, unique_cap)
    return attend_rows(q, keys, values, ids, history)


def batch_topk(act, budget):
    """Positive global Top-k with the flat-index tie rule (core.py:13-26):
    values above the budget-th largest tau (and > 0), then values equal to a
    positive tau in ascending flat index up to the budget."""
    flat = act.reshape(-1)
    budget = min(int(budget), flat.numel())
    if budget == 0:
        return torch.zeros(0, dtype=torch.long)
    tau = torch.topk(flat, budget, sorted=False).values.min()
    above = torch.nonzero((flat > tau) & (flat > 0)).flatten()
    if tau > 0:
        at = torch.nonzero(flat == tau).flatten()[:budget - above.numel()]
        return torch.cat((above, at))
    return above


def append_block(counts, mean, var, lists, history, center, new_keys, W, b, key_scale, key_mean=8):
    """append_index (core.py:186-201) of one group: the block is encoded with
    the ORIGINAL center (relu(x W^T + b), x = (k - center) / scale), its
    BatchTopK memberships (budget len(block) * key_mean) summarised per bucket
    (two-pass population moments of the original keys, a Python loop over the
    buckets as in core.py:82-88), and Chan-merged into (counts, mean, var);
    the block's lists are appended with the +history offset.  Returns the
    new (counts, mean, var, lists)."""
    keys = new_keys.float()
    F = W.shape[0]
    act = torch.nn.functional.linear((keys - center) / key_scale, W.float(), b.float()).relu()
    flat = batch_topk(act, keys.shape[0] * key_mean)
    tok, feat = flat // F, flat % F
    new_lists = [tok[feat == f].sort().values for f in range(F)]
    n_new = torch.tensor([len(x) for x in new_lists], dtype=torch.long)
    m_new = torch.zeros(F, keys.shape[1])
    v_new = torch.zeros_like(m_new)
    for f, members in enumerate(new_lists):
        if len(members):
            rows = keys[members]
            m_new[f] = rows.mean(dim=0)
            v_new[f] = (rows - m_new[f]).square().mean(dim=0)
    a, c = counts.float(), n_new.float()
    tot = a + c
    den = tot.clamp_min(1)
    m = (a[:, None] * mean + c[:, None] * m_new) / den[:, None]
    v = (a[:, None] * var + c[:, None] * v_new) / den[:, None]
    v += ((a * c) / den.square())[:, None] * (mean - m_new).square()
    merged = [torch.cat((old, fresh + history)) for old, fresh in zip(lists, new_lists)]
    return tot.long(), m, v, merged
