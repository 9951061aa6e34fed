"""MI355X-native counterpart of `prismkv.core` (src/prismkv/core.py): the
same names, arguments, return values and error messages, run on this
package's HIP kernels.

The kernels are specialised to the native geometry of the decode path
(src/prismkv/native8b.py:42-43): head_dim 128, F = 3000 buckets, GQA groups
of 4 query heads, on the device.  Like the reference, which computes on
`.float()` of its inputs, keys / queries / values may be of any float dtype:
bf16 inputs run the bf16 kernels, any other dtype is taken as `.float()`
(exact for fp16, the reference's own rounding for fp64) and runs the fp32
entry points, and outputs come back in the input's dtype.  Inputs of another
geometry raise NotImplementedError; there is no CPU path.

A FeatureIndex made here carries its device tables (tiled moments, bucket
sizes, membership bitmap) in `index.native`, so routing, selection and
`append_index` reuse them; an index made elsewhere (lists on the host, say)
gets them built on first use.  Returned lists are ascending int64 tensors on
the keys' device, like the reference's.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from .native8b import (CHUNK, CHUNKS, DIM, ERR_WAIT, ERROR_MESSAGES, FEATURES, HEADS, PADDED, TOPK, FeatureIndex,
                       bitmap_row_words, tile_moments, untile_moments)
from .weights import SharedSAE

__all__ = ["FeatureIndex", "SharedSAE", "positive_global_topk", "summarize", "build_index", "bucket_scores",
           "select_buckets", "attend", "append_index"]

MAX_KEYS = 1 << 20  # rows of one build / topk call (flat indices stay below 2^32)
MAX_BLOCK = 4096    # keys of one append_index block
ATTEND_SPLITS = 32


def _native(cond, what):
    if not cond:
        raise NotImplementedError(f"the MI355X path is specialised to {what}")


def _lib_():
    lib = _lib.load()
    if lib.missing:
        raise RuntimeError(f"{lib.path.name} lacks entry points {lib.missing}; rebuild it")
    return lib


def _stream():
    return torch.cuda.current_stream().cuda_stream


_work_cache: dict = {}


def _work(name, nbytes, device):
    """A zero-filled workspace kept per (entry point, device): for entry points
    whose kernels leave their whole workspace zeroed, so a larger buffer from
    an earlier call serves any later size."""
    key = (name, str(device))
    buf = _work_cache.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = _work_cache[key] = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=device)
    return buf


def _fresh_work(nbytes, device):
    """A new zero-filled workspace of its own for one build or update, whose
    activations stay readable in it (index.native keeps no workspace)."""
    return torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=device)


@dataclass
class NativeTables:
    """One group's device tables: moments f32 [1,94,256,32], n i32 [1,3008],
    bits i32 [1,3000,row_words] for `capacity` tokens."""

    moments: torch.Tensor
    n: torch.Tensor
    bits: torch.Tensor
    row_words: int
    capacity: int

    @classmethod
    def empty(cls, capacity, device):
        rw = bitmap_row_words(capacity)
        return cls(torch.zeros(1, CHUNKS, 2 * DIM, CHUNK, device=device),
                   torch.zeros(1, PADDED, dtype=torch.int32, device=device),
                   torch.zeros(1, FEATURES, rw, dtype=torch.int32, device=device), rw, capacity)

    def widened(self, capacity):
        """A copy with room for `capacity` tokens (the original stays as it is)."""
        out = NativeTables.empty(max(capacity, self.capacity), self.n.device)
        out.moments.copy_(self.moments)
        out.n.copy_(self.n)
        out.bits[:, :, :self.row_words] = self.bits
        return out


def _csr(lists, device):
    lengths = [len(x) for x in lists]
    ids = torch.cat([torch.as_tensor(x).reshape(-1) for x in lists]).to(device=device, dtype=torch.int32) \
        if sum(lengths) else torch.zeros(1, dtype=torch.int32, device=device)
    offsets = torch.zeros(FEATURES + 1, dtype=torch.int64)
    offsets[1:] = torch.tensor(lengths, dtype=torch.int64).cumsum(0)
    return ids.reshape(1, -1).contiguous(), offsets.to(device=device, dtype=torch.int32).reshape(1, -1)


def _bits_from_lists(tables, lists, device):
    ids, offsets = _csr(lists, device)
    _lib_().call("prismkv_build_bits", ids.data_ptr(), offsets.data_ptr(), tables.bits.data_ptr(), 1, ids.shape[1],
                 tables.row_words, stream=_stream())


def _tables(index):
    """The index's device tables, built from its fields on first use."""
    t = getattr(index, "native", None)
    if t is not None:
        return t
    device = index.mean.device
    _native(device.type == "cuda", "indices on the device")
    _native(tuple(index.mean.shape) == (FEATURES, DIM), "F = 3000 buckets of head_dim 128")
    t = NativeTables.empty(index.history, device)
    t.n[0, :FEATURES] = torch.as_tensor(index.counts).to(device=device, dtype=torch.int32)
    t.moments.copy_(tile_moments(index.mean[None].float(), index.variance[None].float()))
    _bits_from_lists(t, index.lists, device)
    index.native = t
    return t


def _lists_from_bits(bits, lo, hi, offset=0):
    """Ascending token lists of bitmap columns [lo, hi), shifted by `offset`."""
    w0, w1 = lo // 32, (hi + 31) // 32
    words = bits[0, :, w0:w1]
    shifts = torch.arange(32, device=bits.device, dtype=torch.int32)
    flags = ((words.unsqueeze(-1) >> shifts) & 1).to(torch.bool).reshape(FEATURES, -1)
    flags = flags[:, lo - 32 * w0:hi - 32 * w0]
    f, t = flags.nonzero(as_tuple=True)
    per = torch.bincount(f, minlength=FEATURES).tolist()
    return list(torch.split(t + (lo + offset), per))


def _native_rows(x, what):
    """Rows of head_dim 128 for the kernels and the entry-point suffix: bf16
    stays bf16 (""), any other float dtype becomes x.float() ("_f32")."""
    _native(x.device.type == "cuda", f"{what} on the device")
    _native(x.dtype.is_floating_point, f"floating-point {what}")
    _native(x.shape[-1] == DIM, "head_dim 128")
    suffix = ""
    if x.dtype != torch.bfloat16:
        x, suffix = x.float(), "_f32"
    x = x if x.stride(-1) == 1 and (x.ndim == 1 or x.stride(-2) == DIM) else x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    return x, suffix


def _check_keys(keys):
    _native(len(keys) <= MAX_KEYS, f"at most {MAX_KEYS} keys per call")
    return _native_rows(keys, "keys")


def _check_sae(sae):
    _native(sae.head_dim == DIM and sae.features == FEATURES, "SAEs of 3000 features over head_dim 128")


# ------------------------------------------------------------------ stage 4

@torch.no_grad()
def positive_global_topk(a: torch.Tensor, count: int):
    """src/prismkv/core.py:13-26 on the device: strict values above the
    budget-th largest (and above 0) in ascending flat index, then ties at a
    positive threshold in ascending flat index up to the budget."""
    if a.ndim != 2 or count < 0:
        raise ValueError("expected a matrix and nonnegative activation budget")
    count = min(int(count), a.numel())
    if count == 0:
        return torch.empty(0, dtype=torch.long, device=a.device)
    _native(a.device.type == "cuda", "activations on the device")
    _native(a.shape[1] == FEATURES, "activation matrices of 3000 buckets")
    _native(a.dtype in (torch.float32, torch.bfloat16, torch.float16), "fp32 / bf16 / fp16 activations")
    _native(a.shape[0] <= MAX_KEYS, f"at most {MAX_KEYS} rows")
    a = a.float().contiguous()  # widening is exact
    if a.data_ptr() % 16:
        a = a.clone()
    lib = _lib_()
    out = torch.empty(count, dtype=torch.long, device=a.device)
    out_len = torch.zeros(1, dtype=torch.int32, device=a.device)
    work = _work("topk", lib.query("prismkv_topk_work_bytes"), a.device)
    lib.call("prismkv_topk", a.data_ptr(), out.data_ptr(), out_len.data_ptr(), work.data_ptr(), a.shape[0], count,
             _lib.nbytes(work), stream=_stream())
    return out[:int(out_len.item())]


@torch.no_grad()
def summarize(keys, lists, center=None):
    """src/prismkv/core.py:76-89: population diagonal moments of the ORIGINAL
    keys over each bucket's list (two passes), center = keys.float().mean(0)
    unless given."""
    n, d = keys.shape
    keys, suffix = _check_keys(keys)
    _native(len(lists) == FEATURES, "3000 bucket lists")
    lib = _lib_()
    t = NativeTables.empty(n, keys.device)
    _bits_from_lists(t, lists, keys.device)
    c = torch.zeros(1, DIM, device=keys.device) if center is None else \
        torch.as_tensor(center).to(device=keys.device, dtype=torch.float32).reshape(1, DIM).clone()
    work = _work("summarize", lib.query("prismkv_summarize_work_bytes", 1), keys.device)
    lib.call("prismkv_summarize" + suffix, keys.data_ptr(), t.bits.data_ptr(), c.data_ptr(), t.n.data_ptr(),
             t.moments.data_ptr(), work.data_ptr(), 1, n, 1 if center is None else 0, keys.stride(0) * n, t.row_words,
             _lib.nbytes(work), stream=_stream())
    mean, var = untile_moments(t.moments)
    counts = torch.tensor([len(x) for x in lists], device=keys.device, dtype=torch.long)
    out = FeatureIndex(n, c[0] if center is None else center, counts, mean[0].contiguous(), var[0].contiguous(),
                       lists)
    out.native = t
    return out


def _encoder(sae, device):
    W = sae.W_enc.detach().to(device=device, dtype=torch.float32).reshape(1, FEATURES, DIM).contiguous()
    b = sae.b_enc.detach().to(device=device, dtype=torch.float32).reshape(1, FEATURES).contiguous()
    return W, b


@torch.no_grad()
def build_index(keys, sae, key_scale, *, center=None):
    """src/prismkv/core.py:92-103 on the device: encode, BatchTopK with the
    budget len(keys) * key_mean, per-bucket ascending lists, summarize."""
    if keys.ndim != 2 or len(keys) == 0 or key_scale <= 0:
        raise ValueError("nonempty [history,head_dim] keys and positive scale required")
    if keys.shape[-1] != sae.head_dim:
        raise ValueError("SAE and attention head dimensions differ")
    _check_sae(sae)
    keys, suffix = _check_keys(keys)
    n, device = len(keys), keys.device
    lib = _lib_()
    t = NativeTables.empty(n, device)
    W, b = _encoder(sae, device)
    scale = torch.tensor([float(key_scale)], dtype=torch.float32, device=device)
    c = torch.zeros(1, DIM, device=device) if center is None else \
        torch.as_tensor(center).to(device=device, dtype=torch.float32).reshape(1, DIM).clone()
    work = _fresh_work(lib.query("prismkv_build_work_bytes", 1, n), device)
    lib.call("prismkv_build" + suffix, keys.data_ptr(), W.data_ptr(), b.data_ptr(), c.data_ptr(), scale.data_ptr(),
             t.bits.data_ptr(), t.n.data_ptr(), t.moments.data_ptr(), work.data_ptr(), 1, 1, n, int(sae.key_mean),
             1 if center is None else 0, keys.stride(0) * n, t.row_words, _lib.nbytes(work), stream=_stream())
    mean, var = untile_moments(t.moments)
    out = FeatureIndex(n, c[0] if center is None else torch.as_tensor(center).to(device), t.n[0, :FEATURES].long(),
                       mean[0].contiguous(), var[0].contiguous(), _lists_from_bits(t.bits, 0, n))
    out.native = t
    return out


@torch.no_grad()
def append_index(index, new_keys, sae, key_scale):
    """src/prismkv/core.py:186-201 on the device: index only the new block
    with the index's ORIGINAL center (BatchTopK budget over the block), merge
    the moments with the reference's formula and operation order, append the
    block's memberships at columns history + t.  The given index is left as
    it is; the result has its own tables."""
    if new_keys.ndim != 2 or len(new_keys) == 0 or key_scale <= 0:
        raise ValueError("nonempty [history,head_dim] keys and positive scale required")
    if new_keys.shape[-1] != sae.head_dim:
        raise ValueError("SAE and attention head dimensions differ")
    _check_sae(sae)
    new_keys, suffix = _check_keys(new_keys)
    N, H, device = len(new_keys), index.history, new_keys.device
    _native(N <= MAX_BLOCK, f"append blocks of at most {MAX_BLOCK} keys")
    lib = _lib_()
    t = _tables(index).widened(H + N)
    W, b = _encoder(sae, device)
    scale = torch.tensor([float(key_scale)], dtype=torch.float32, device=device)
    c = torch.as_tensor(index.center).to(device=device, dtype=torch.float32).reshape(1, DIM).contiguous()
    work = _fresh_work(lib.query("prismkv_update_work_bytes", 1, N), device)
    # the kernels read K rows [H, H + N) of the buffer: address the block as those rows
    row_bytes = DIM * new_keys.element_size()
    base = new_keys.data_ptr() - H * row_bytes
    lib.call("prismkv_update" + suffix, base, W.data_ptr(), b.data_ptr(), c.data_ptr(), scale.data_ptr(),
             t.bits.data_ptr(), t.n.data_ptr(), t.moments.data_ptr(), work.data_ptr(), 1, H, N, int(sae.key_mean),
             (H + N) * DIM, t.row_words, _lib.nbytes(work), stream=_stream())
    mean, var = untile_moments(t.moments)
    new_lists = _lists_from_bits(t.bits, H, H + N)
    lists = [torch.cat((torch.as_tensor(old).to(device=device, dtype=torch.long), new))
             for old, new in zip(index.lists, new_lists)]
    out = FeatureIndex(H + N, index.center, t.n[0, :FEATURES].long(), mean[0].contiguous(), var[0].contiguous(),
                       lists)
    out.native = t
    return out


# ------------------------------------------------------------------ stages 1-3

def _check_q(q):
    """[1, 4, 128] queries for the kernels and the entry-point suffix."""
    _native(tuple(q.shape) == (HEADS, DIM), "GQA groups of 4 query heads of head_dim 128")
    q, suffix = _native_rows(q, "queries")
    return q.reshape(1, HEADS, DIM), suffix


QA_WIDTH = 64  # the q_activation selection: up to 4 heads x 16 buckets


def _route_qact(q, index, sae, query_scale, scores):
    t = _tables(index)
    q1, suffix = _check_q(q)
    _check_sae(sae)
    lib = _lib_()
    device = q1.device
    W, b = _encoder(sae, device)
    qs = torch.tensor([float(query_scale)], dtype=torch.float32, device=device)
    features = torch.zeros(1, QA_WIDTH, dtype=torch.int64, device=device)
    valid = torch.zeros(1, QA_WIDTH, device=device)
    raw = torch.zeros(1, dtype=torch.int32, device=device)
    work = _work("route_qact", lib.query("prismkv_route_qact_work_bytes", 1), device)
    lib.call("prismkv_route_qact" + suffix, q1.data_ptr(), W.data_ptr(), b.data_ptr(), qs.data_ptr(), t.n.data_ptr(),
             work.data_ptr(), features.data_ptr(), valid.data_ptr(), raw.data_ptr(), scores.data_ptr(), 1,
             _lib.nbytes(work), stream=_stream())
    return t, features, valid, raw


def _route(q, index, scores):
    t = _tables(index)
    q1, suffix = _check_q(q)
    lib = _lib_()
    device = q1.device
    features = torch.zeros(1, TOPK, dtype=torch.int64, device=device)
    valid = torch.zeros(1, TOPK, device=device)
    raw = torch.zeros(1, dtype=torch.int32, device=device)
    work = _work("route", lib.query("prismkv_route_work_bytes", 1), device)
    lib.call("prismkv_route_scores" + suffix, q1.data_ptr(), t.moments.data_ptr(), t.n.data_ptr(), work.data_ptr(),
             features.data_ptr(), valid.data_ptr(), raw.data_ptr(), scores.data_ptr(), 1, _lib.nbytes(work),
             stream=_stream())
    return t, features, valid, raw


def _check_router(router="moments", sae=None, query_scale=None, query_topk=16,
                  terms=("count", "mean", "variance")):
    """The argument checks of core.py:118-120,131-132, then the native limits."""
    if router == "moments":
        if not terms or set(terms) - {"count", "mean", "variance"}:
            raise ValueError("specify exact estimator components")
        _native(set(terms) == {"count", "mean", "variance"}, "the full count/mean/variance estimator")
    elif router != "q_activation" or sae is None or query_scale is None or query_scale <= 0:
        raise ValueError("q_activation requires SAE and saved positive query scale")
    _native(query_topk == TOPK, "16 buckets per query (router q_activation) or in all (router moments)")
    return router


@torch.no_grad()
def bucket_scores(q, index, *, router="moments", sae=None, query_scale=None, query_topk=16,
                  terms=("count", "mean", "variance")):
    """src/prismkv/core.py:106-139 on the device.  "moments": the head-mean
    softmax scores of the 3000 buckets and the live buckets of the top 16
    (score descending, bucket ascending on ties).  "q_activation": the
    scores of the 4 queries' top-16 SAE activations, normalised per query,
    and every live bucket of positive score (up to 64), same order."""
    _check_router(router, sae, query_scale, query_topk, terms)
    scores = torch.zeros(1, FEATURES, device=q.device)
    if router == "moments":
        _, features, valid, _ = _route(q, index, scores)
    else:
        _, features, valid, _ = _route_qact(q, index, sae, query_scale, scores)
    return scores[0], features[0][valid[0] > 0]


@torch.no_grad()
def select_buckets(q, index, *, unique_cap=None, **kwargs):
    """src/prismkv/core.py:142-167 on the device: the union of the selected
    buckets' lists (ascending int64 ids) and meta (features, raw, unique,
    limit, candidate_buckets, scores); with a cap, a ranked bucket whose new
    ids would overflow floor(history * unique_cap) is skipped.  Both routers
    of bucket_scores."""
    if unique_cap is not None and not 0 <= unique_cap <= 1:
        raise ValueError("unique_cap must be a fraction in [0,1]")
    router = _check_router(**kwargs)
    H = index.history
    scores = torch.zeros(1, FEATURES, device=q.device)
    if router == "q_activation":
        t, features, valid, raw = _route_qact(q, index, kwargs["sae"], kwargs["query_scale"], scores)
        width = QA_WIDTH
    else:
        t, features, valid, raw = _route(q, index, scores)
        width = TOPK
    candidates = int((valid[0] > 0).sum())
    limit = H if unique_cap is None else math.floor(H * unique_cap)
    lib = _lib_()
    if unique_cap is not None:
        lib.call("prismkv_select_cap_n", t.bits.data_ptr(), t.n.data_ptr(), features.data_ptr(), valid.data_ptr(),
                 raw.data_ptr(), 1, H, limit, t.row_words, width, stream=_stream())
    ids = torch.zeros(1, max(H, 1), dtype=torch.int32, device=q.device)
    count = torch.zeros(1, dtype=torch.int32, device=q.device)
    work = _work("union", lib.query("prismkv_union_work_bytes", 1, H), q.device)
    lib.call("prismkv_union_n", t.bits.data_ptr(), features.data_ptr(), valid.data_ptr(), work.data_ptr(),
             ids.data_ptr(), count.data_ptr(), 1, H, t.row_words, ids.shape[1], width, _lib.nbytes(work),
             stream=_stream())
    n = int(count.item())
    if int(work[:4].view(torch.int32).item()):  # a bounded wait of the union gave up
        work.zero_()
        raise RuntimeError("prismkv_union_n: a bounded inter-workgroup wait gave up; the workspace was reset")
    kept = features[0][valid[0] > 0].tolist()
    assert n <= limit
    return ids[0, :n].long(), dict(features=kept, raw=int(raw.item()), unique=n, limit=limit,
                                   candidate_buckets=candidates, scores=scores[0])


@torch.no_grad()
def attend(q, keys, values, old_ids, history):
    """src/prismkv/core.py:170-183 on the device: exact softmax attention of
    the 4 heads over the given history rows plus the dense tail
    [history, len(keys)), fp32 accumulation, output in q's dtype."""
    if keys.shape != values.shape or not 0 <= history <= len(keys):
        raise ValueError("invalid KV/history")
    if len(old_ids) and (old_ids.min() < 0 or old_ids.max() >= history):
        raise ValueError("old_ids must address old history only")
    if len(old_ids.unique()) != len(old_ids):
        raise ValueError("deduplicate history before attention")
    if len(old_ids) + len(keys) - history == 0:
        return q.new_zeros(q.shape)
    _native(tuple(q.shape) == (HEADS, DIM), "GQA groups of 4 query heads of head_dim 128")
    # q @ K^T and P @ V of core.py:182-183 on .float() of each operand: all
    # bf16 runs the bf16 kernel, anything else the fp32 one on fp32 copies
    for x, name in ((q, "queries"), (keys, "keys"), (values, "values")):
        _native(x.dtype.is_floating_point, f"floating-point {name}")
    bf16 = all(x.dtype == torch.bfloat16 for x in (q, keys, values))
    dtype, suffix = (torch.bfloat16, "") if bf16 else (torch.float32, "_f32")
    q1, keys, values = (_native_rows(x.to(dtype), name)[0] for x, name in
                        ((q, "queries"), (keys, "keys"), (values, "values")))
    q1 = q1.reshape(1, HEADS, DIM)
    L = len(keys)
    lib = _lib_()
    # an id row as wide as the history (the entry point's row stride), first len(old_ids) used
    ids = torch.zeros(1, max(history, len(old_ids), 1), dtype=torch.int32, device=q.device)
    ids[0, :len(old_ids)] = old_ids.to(device=q.device, dtype=torch.int32)
    count = torch.tensor([len(old_ids)], dtype=torch.int32, device=q.device)
    out = torch.empty(1, HEADS, DIM, dtype=dtype, device=q.device)
    work = _work("attend", lib.query("prismkv_attend_work_bytes", 1, ATTEND_SPLITS), q.device)
    lib.call("prismkv_attend" + suffix, q1.data_ptr(), keys.data_ptr(), values.data_ptr(), ids.data_ptr(),
             count.data_ptr(), work.data_ptr(), out.data_ptr(), 1, history, L - history, L * DIM, L * DIM,
             ids.shape[1], ATTEND_SPLITS, _lib.nbytes(work), stream=_stream())
    code = int(work[:4].view(torch.int32).item())
    if code:  # a bounded wait of the attention gave up (ids were checked above)
        work.zero_()
        raise RuntimeError(f"prismkv_attend{suffix}: {ERROR_MESSAGES.get(code, ERROR_MESSAGES[ERR_WAIT])}; "
                           "the workspace was reset")
    return out[0].to(q.dtype)
