"""Hugging Face attention backend for unpadded, batch-one causal decoding
through the MI355X routed-decode path -- the native counterpart of
src/prismkv/hf_reference.py:65-240 (`HFReference`): the same constructor
arguments, methods (`begin_request`, `prefill`, `close`, `generate`,
`records`) and checks with the same messages, so a caller switches backends
without code changes.

Prefill runs the model's own attention (SDPA or eager).  At a layer's first
decode step its 8 KV groups are indexed on the device from the prefix keys
(the reference's lazy `build_index`, hf_reference.py:196-198); every decode
step then indexes the complete old tail blocks (the update trigger of
:205-211) and decodes all 8 groups of the layer in one `Native8B` call.  The
current token and the un-indexed tail are attended densely, as in the
reference.

Native specialisation (NotImplementedError otherwise): Qwen3 attention with 8
KV heads x 4 query heads, head_dim 128, bf16 activations, 16 selected buckets
(per query for router "q_activation").  `unique_cap` maps to
`Native8B.unique_cap`; mode "all_read" (the dense control) runs the model's
own attention over the whole cache.

Records keep the reference's per-(layer, group) fields, including the
`detailed_records` ones (old_unique, old_raw, generated_indexed_unique,
generated_indexed_raw, initial_history, hf_reference.py:216-231); they are
computed on the device as device tensors and read back when `records` is
first accessed after a step, so decoding never synchronises.

`DecodeGraph` (no reference counterpart; the role of the SM90 runner's
captured step, kernels/cuda_sm90/single.py:211-233) decodes from a
transformers `StaticCache`: the model's whole one-token forward, every
layer's decode reading its tail length from the device, is captured once in
a HIP graph and replayed token after token, with or without a unique cap;
the lazy builds and the update policy run eagerly between replays, and the
step is recaptured whenever a layer's history moves.
"""
from __future__ import annotations

import importlib
import math
from contextlib import contextmanager
from dataclasses import dataclass

import torch

from .native8b import DIM, FEATURES, GROUPS, HEADS, MAX_BLOCK, Native8B
from .weights import Encoder, layer_tables  # noqa: F401  (Encoder re-exported: reference name)

BACKEND = "prismkv_native"
BACKEND_EAGER = "prismkv_native_eager"
ATTENTION_MODULES = ("Qwen3Attention", "Qwen3_5Attention")


def _route_to_session(module, q, k, v, attention_mask, **kwargs):
    """The registered attention function: hands the call to the session
    attached to the module (the reference's `_dispatch`, same message)."""
    owner = getattr(module, "_prismkv_session", None)
    if owner is None:
        raise RuntimeError("PrismKV backend selected without an attached session")
    return owner.forward(module, q, k, v, attention_mask, **kwargs)


@dataclass
class _Hooked:
    """An attention module served by a session and what it ran before."""
    module: object
    config: object
    implementation: str
    original: object


def _find_attention(model):
    """{layer: _Hooked} for every standard attention module of the model,
    rejecting what the reference rejects (same messages)."""
    hooked = {}
    for module in filter(lambda m: type(m).__name__ in ATTENTION_MODULES, model.modules()):
        if hasattr(module, "_prismkv_session"):
            raise ValueError("model already has a reference session")
        if module.layer_idx in hooked:
            raise ValueError("duplicate attention-layer IDs")
        impl = module.config._attn_implementation
        if impl not in ("sdpa", "eager"):
            raise ValueError("reference adapter is validated for SDPA/eager prefill only")
        # the module's own namespace (decorators may wrap forward's globals)
        names = vars(importlib.import_module(type(module).__module__))
        original = names["eager_attention_forward"] if impl == "eager" else names["ALL_ATTENTION_FUNCTIONS"][impl]
        hooked[module.layer_idx] = _Hooked(module, module.config, impl, original)
    return hooked


def _register_backends():
    """Both backend names: eager prefill needs an explicit causal mask,
    which SDPA's mask function may elide."""
    from transformers import AttentionInterface, AttentionMaskInterface
    from transformers.masking_utils import eager_mask, sdpa_mask
    for name, mask in ((BACKEND, sdpa_mask), (BACKEND_EAGER, eager_mask)):
        AttentionInterface.register(name, _route_to_session)
        AttentionMaskInterface.register(name, mask)


def _additive_mask(blocked, dtype):
    """[steps, keys] boolean "not visible" -> an additive [1, 1, steps, keys] mask."""
    mask = torch.zeros((1, 1) + tuple(blocked.shape), dtype=dtype, device=blocked.device)
    return mask.masked_fill_(blocked[None, None], float("-inf"))


def _check_call(q, k, v, kwargs):
    """The reference's argument checks (hf_reference.py:153-164, same messages)."""
    if q.shape[0] != 1 or k.shape[0] != 1:
        raise NotImplementedError("reference adapter supports unpadded batch-one requests")
    if q.shape[-2] < 1 or q.shape[-1] != k.shape[-1] or k.shape != v.shape:
        raise ValueError("invalid QKV shapes")
    d = q.shape[-1]
    if not math.isclose(kwargs.get("scaling", 1 / math.sqrt(d)), 1 / math.sqrt(d)):
        raise NotImplementedError("nonstandard attention scale")
    if kwargs.get("sliding_window") is not None or kwargs.get("softcap") is not None:
        raise NotImplementedError("sliding-window/soft-capped attention is outside this adapter")
    if kwargs.get("dropout", 0) != 0:
        raise ValueError("inference only: disable dropout")


def _check_unpadded(attention_mask, total):
    """On an unpadded causal request the last query sees every key."""
    if attention_mask is None:
        return
    if attention_mask.ndim != 4:
        raise NotImplementedError("padding/arbitrary attention masks are unsupported")
    last = attention_mask[..., -1, :total]
    hidden = ~last if last.dtype == torch.bool else last != 0
    if bool(hidden.any()):
        raise NotImplementedError("padding/arbitrary attention masks are unsupported")


def _native_geometry(q, k):
    """(groups, queries) of a one-token decode call the native path serves."""
    if q.shape[-2] != 1:
        raise NotImplementedError("decode reference is one token per forward")
    groups, queries = k.shape[1], q.shape[1]
    if queries % groups:
        raise ValueError("Q heads must form equal-sized KV groups")
    if groups != GROUPS or queries != GROUPS * HEADS or q.shape[-1] != DIM or q.dtype != torch.bfloat16:
        raise NotImplementedError("the native path decodes 8 KV groups x 4 query heads, d=128, in bf16")
    return groups, queries


def _popcount32(words):
    """Set bits of each 32-bit word (int32 tensor) as int64."""
    x = words.to(torch.int64) & 0xFFFFFFFF
    x = x - ((x >> 1) & 0x55555555)
    x = (x & 0x33333333) + ((x >> 2) & 0x33333333)
    x = (x + (x >> 4)) & 0x0F0F0F0F
    return ((x * 0x01010101) & 0xFFFFFFFF) >> 24


def _old_unique_raw(op, prefix):
    """Per group, on the device: the selected ids below `prefix` (ids are
    ascending) and the members below `prefix` summed over the kept buckets
    (their bitmap words before the prefix), hf_reference.py:220-225."""
    device = op.ids.device
    live = torch.arange(op.ids.shape[1], device=device)[None] < op.count[:, None].long()
    old_unique = ((op.ids < prefix) & live).sum(1)
    full, rest = divmod(int(prefix), 32)
    rows = op.bits[torch.arange(GROUPS, device=device)[:, None], op.features.clamp(0, FEATURES - 1)]
    rows = rows[..., :full + (1 if rest else 0)]
    if rest:
        rows = rows.clone()
        rows[..., full] &= (1 << rest) - 1
    per_bucket = _popcount32(rows).sum(-1)
    old_raw = (per_bucket * (op.valid > 0)).sum(1)
    return old_unique, old_raw


class _Records:
    """Decode records as device tensors until read (no synchronisation per step)."""

    def __init__(self, mode, detailed):
        self.mode, self.detailed = mode, detailed
        self.done, self.pending = [], []

    def sparse(self, layer, op, total, prefix):
        entry = dict(layer=layer, history=op.history, total=total, prefix=prefix, unique=op.count.clone(),
                     raw=op.raw.clone(), buckets=(op.valid > 0).sum(1))
        if self.detailed:
            entry["old_unique"], entry["old_raw"] = _old_unique_raw(op, prefix)
        self.pending.append(entry)

    def dense(self, layer, prefix, total):
        n = torch.full((GROUPS,), prefix)
        self.pending.append(dict(layer=layer, history=prefix, total=total, prefix=prefix, unique=n, raw=n,
                                 buckets=torch.zeros(GROUPS, dtype=torch.long), old_unique=n, old_raw=n))

    def read(self):
        for e in self.pending:
            cols = {key: e[key].tolist() for key in ("unique", "raw", "buckets", "old_unique", "old_raw") if key in e}
            for g in range(GROUPS):
                rec = dict(layer=e["layer"], group=g, history=e["history"], unique=cols["unique"][g],
                           raw=cols["raw"][g], buckets=cols["buckets"][g], tail=e["total"] - e["history"],
                           routing_policy=self.mode)
                if self.detailed:
                    old_u, old_r = cols["old_unique"][g], cols["old_raw"][g]
                    rec.update(initial_history=e["prefix"], old_unique=old_u, old_raw=old_r,
                               generated_indexed_unique=rec["unique"] - old_u,
                               generated_indexed_raw=rec["raw"] - old_r)
                self.done.append(rec)
        self.pending = []
        return self.done


class HFNative:
    """Stateful all-group adapter; one session per model, one request at a
    time.  `capacity_step` is the token granularity by which a layer's index
    capacity grows as the request gets longer."""

    def __init__(self, model, encoders, *, mode="sparse", router="moments", selected_buckets=16, unique_cap=None,
                 update_interval=4096, detailed_records=False, capacity_step=8192, library=None):
        # the reference's policy checks (hf_reference.py:77-84), then the native limits
        if mode not in ("sparse", "all_read"):
            raise ValueError("mode must be sparse or all_read")
        if router not in ("moments", "q_activation") or selected_buckets <= 0:
            raise ValueError("unsupported router/bucket count")
        if unique_cap is not None and not 0 <= unique_cap <= 1:
            raise ValueError("unique cap must be a fraction")
        if update_interval <= 0:
            raise ValueError("positive update interval required")
        if mode == "sparse" and selected_buckets != 16:
            raise NotImplementedError("the native path selects 16 buckets (per query for q_activation)")
        if not 1 <= update_interval <= MAX_BLOCK:
            raise NotImplementedError(f"the native update indexes blocks of at most {MAX_BLOCK} keys")
        hooked = _find_attention(model)
        wanted = {(layer, g) for layer, h in hooked.items() for g in range(h.config.num_key_value_heads)}
        if not hooked or set(encoders) != wanted:
            raise ValueError(f"provide exactly all standard-attention KV encoders; missing={wanted - set(encoders)}, "
                             f"extra={set(encoders) - wanted}")
        self.model, self.encoders = model, encoders
        self.mode, self.router = mode, router
        self.selected_buckets, self.unique_cap = selected_buckets, unique_cap
        self.update_interval, self.force_prefill = update_interval, False
        self.detailed_records = detailed_records
        self.capacity_step, self.library = int(capacity_step), library
        self._hooked = hooked
        self.modules = {layer: h.module for layer, h in hooked.items()}
        self.original = {layer: h.original for layer, h in hooked.items()}
        self._tables = {}    # layer -> encoder tables on the model's device
        self._static = None  # the DecodeGraph driving a static cache, if any
        _register_backends()  # only after every non-mutating check passed
        for h in hooked.values():
            h.module._prismkv_session = self
            h.config._attn_implementation = BACKEND_EAGER if h.implementation == "eager" else BACKEND
        self.begin_request()

    # ------------------------------------------------------------ lifecycle

    def begin_request(self):
        if getattr(self, "_static", None) is not None:  # the finished request's steps join its records
            self._static.flush_records()
        self.prefix_lengths, self.ops = {}, {}
        self._log = _Records(self.mode, self.detailed_records)

    @contextmanager
    def prefill(self):
        """Explicitly mark chunked prefill, including one-token chunks."""
        outer, self.force_prefill = self.force_prefill, True
        try:
            yield self
        finally:
            self.force_prefill = outer

    def close(self):
        """Detach from the model and restore every attention implementation."""
        for h in self._hooked.values():
            if getattr(h.module, "_prismkv_session", None) is self:
                del h.module._prismkv_session
            h.config._attn_implementation = h.implementation
        self.ops.clear()

    def generate(self, *args, **kwargs):
        """Reset for a new model.generate call/cache."""
        if kwargs.get("past_key_values") is not None:
            raise ValueError("use manual model calls and session state for an existing cache")
        self.begin_request()
        return self.model.generate(*args, **kwargs)

    @property
    def records(self):
        """Per-(layer, group) decode records in the reference's fields (reads
        the pending device tensors back; raises if a decode's bounded wait
        gave up)."""
        if self._static is not None:
            self._static.flush_records()
        if self._log.pending:
            torch.cuda.synchronize()
            self.check_errors()
        return self._log.read()

    def check_errors(self):
        """RuntimeError if a bounded wait of any layer's launches gave up
        (reads host-mapped words; no synchronisation)."""
        for op in self.ops.values():
            op.check_errors()

    # ------------------------------------------------------------ indices

    def _capacity(self, total):
        if self._static is not None:  # a static cache never outgrows its buffers
            return self._static.max_length
        step = max(self.capacity_step, self.update_interval)
        return (total // step + 1) * step

    def _index(self, layer, K, total):
        """The layer's Native8B: built from the prefix keys at its first decode
        step, its capacity grown as the request gets longer."""
        op = self.ops.get(layer)
        if op is None:
            if layer not in self._tables:
                self._tables[layer] = layer_tables(self.encoders, layer, GROUPS, K.device)
            W, b, scale, key_mean = self._tables[layer]
            op = Native8B.from_keys(K, self.prefix_lengths[layer], W, b, scale, key_mean, self.library,
                                    capacity=self._capacity(total), unique_cap=self.unique_cap)
            if self.router == "q_activation":  # the same SAEs encode the queries (hf_reference.py:213-215)
                op.set_query_encoders(W, b, [float(self.encoders[(layer, g)].query_scale) for g in range(GROUPS)])
                op.router = "q_activation"
            self.ops[layer] = op
        elif total > op.capacity:
            op.grow(self._capacity(total))
        return op

    # ------------------------------------------------------------ forward

    def _starts_prefill(self, layer, steps):
        return self.force_prefill or steps > 1 or layer not in self.prefix_lengths

    @torch.no_grad()
    def forward(self, module, q, k, v, attention_mask, **kwargs):
        _check_call(q, k, v, kwargs)
        if self._static is not None:
            return self._forward_static(module, q, k, v, attention_mask, **kwargs)
        layer, total, steps = module.layer_idx, k.shape[-2], q.shape[-2]
        _check_unpadded(attention_mask, total)
        if self._starts_prefill(layer, steps):
            # a new prefix: forget the layer's index, run the model's attention
            self.prefix_lengths[layer] = total
            self.ops.pop(layer, None)
            if attention_mask is None and 1 < steps < total:
                # a cached chunk: query i sits at position total - steps + i
                blocked = torch.ones(steps, total, dtype=torch.bool, device=q.device).triu_(total - steps + 1)
                attention_mask = _additive_mask(blocked, q.dtype)
            return self.original[layer](module, q, k, v, attention_mask, **kwargs)
        _, queries = _native_geometry(q, k)
        prefix = self.prefix_lengths[layer]
        if self.mode == "all_read":
            self._log.dense(layer, prefix, total)
            return self.original[layer](module, q, k, v, attention_mask, **kwargs)
        K, V = k[0], v[0]
        if K.stride(-1) != 1 or K.stride(-2) != DIM:
            K, V = K.contiguous(), V.contiguous()
        op = self._index(layer, K, total)
        op.catch_up(K, total, self.update_interval)
        out = op(q[0, :, 0].reshape(GROUPS, HEADS, DIM).contiguous(), K, V)
        self._log.sparse(layer, op, total, prefix)
        return out.reshape(1, 1, queries, q.shape[-1]), None

    def _forward_static(self, module, q, k, v, attention_mask, **kwargs):
        """forward() over a StaticCache: K/V are the whole preallocated buffers
        and the positions come from `position_ids`.  Prefill (eager) runs the
        model's own attention under an explicit causal mask; a decode step
        launches the layer's decode with the tail length computed on the
        device, so it can be captured and replayed."""
        layer, steps = module.layer_idx, q.shape[-2]
        pos = kwargs.get("position_ids")
        if pos is None:
            raise ValueError("a static-cache forward passes position_ids")
        pos = pos.reshape(-1)
        if self._starts_prefill(layer, steps):
            if q.is_cuda and torch.cuda.is_current_stream_capturing():
                raise RuntimeError("prefill cannot be captured")
            self.prefix_lengths[layer] = int(pos[-1]) + 1
            self.ops.pop(layer, None)
            if attention_mask is None:  # key j is visible to the query at position p iff j <= p
                blocked = torch.arange(k.shape[-2], device=q.device)[None] > pos.to(q.device)[:, None]
                attention_mask = _additive_mask(blocked, q.dtype)
            return self.original[layer](module, q, k, v, attention_mask, **kwargs)
        _, queries = _native_geometry(q, k)
        op = self.ops.get(layer)
        if op is None:
            raise RuntimeError("static-cache decode steps run through DecodeGraph")
        tail = (pos[-1:] + 1 - op.history).to(torch.int32)
        out = op(q[0, :, 0].reshape(GROUPS, HEADS, DIM).contiguous(), k[0], v[0], tail=tail)
        self._static._record(layer, op)
        return out.reshape(1, 1, queries, q.shape[-1]), None


class DecodeGraph:
    """One-token decode steps of `session.model` from a transformers
    StaticCache, captured in a HIP graph and replayed.  Create it before
    the prefill (the session then runs every forward over the static
    buffers), prefill the prompt through the model with position_ids, then
    call it once per generated token.

    Each call takes the next token id ([1, 1] int64 on the model's device)
    and returns the last-position logits (a static buffer, overwritten by
    the next step).  Before a step, on the host: every layer without an
    index is built from its prefix (hf_reference.py:196-198) and every
    index absorbs the complete old tail blocks (the update loop of
    :205-211); if any history moved, the step is captured again.  The
    capture covers the model's forward with the cache write, RoPE and every
    layer's decode (tail length = position + 1 - history, computed on the
    device): one launch per layer, or with a unique cap the route, the
    budgeted walk and the union + attention launch.  With graph=False every
    step runs eagerly through the same code.  Sparse mode and the moments
    router only.

    Records (the session's `records`, hf_reference.py:216-231): each step's
    decode writes its count, raw and selection of every layer into a device
    ring of `record_steps` slots, indexed by the step's position on the
    device, inside the captured step; the host notes each step's histories
    and reads the ring back when `records` is read or the ring is full (one
    synchronisation per `record_steps` steps).  The detailed fields are not
    kept here (detailed_records raises)."""

    def __init__(self, session, cache, *, graph=True, record_steps=1024):
        if session.mode != "sparse" or session.router != "moments":
            raise NotImplementedError("DecodeGraph drives the fused decode: sparse mode, moments router")
        if session.detailed_records:
            raise NotImplementedError("DecodeGraph keeps the basic records (detailed_records=False)")
        if session._static is not None:
            raise ValueError("the session already drives a static cache")
        if int(record_steps) < 1:
            raise ValueError("record_steps must be positive")
        device = next(session.model.parameters()).device
        self.session, self.cache, self.position = session, cache, None
        self.max_length = int(cache.max_cache_len)
        self.use_graph = bool(graph)
        self.ids = torch.zeros((1, 1), dtype=torch.long, device=device)
        self.pos = torch.zeros((1, 1), dtype=torch.long, device=device)
        self.graph, self.logits, self.stale = None, None, True
        self.eager_steps = 0
        self.record_steps = int(record_steps)
        self._slot = torch.zeros(1, dtype=torch.long, device=device)  # ring slot of the current step
        self._rings = {}   # layer -> device ring of (count, raw, valid) per step
        self._steps = []   # (position, {layer: history}) of the steps in the rings, oldest first
        session._static = self

    def close(self):
        self.flush_records()
        if self.session._static is self:
            self.session._static = None
        self.graph = self.logits = None

    def _record(self, layer, op):
        """Copies the layer's count / raw / valid into the step's ring slot
        (device-side index, so a captured step records every replay)."""
        ring = self._rings.get(layer)
        if ring is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("record rings are created by an eager step")
            R, dev = self.record_steps, op.out.device
            ring = self._rings[layer] = (torch.zeros(R, GROUPS, dtype=torch.int32, device=dev),
                                         torch.zeros(R, GROUPS, dtype=torch.int32, device=dev),
                                         torch.zeros(R, *op.valid.shape, dtype=op.valid.dtype, device=dev))
        for dst, src in zip(ring, (op.count, op.raw, op.valid)):
            dst.index_copy_(0, self._slot, src[None])

    def flush_records(self):
        """Moves the recorded steps into the session's records (synchronises)."""
        if not self._steps:
            return
        torch.cuda.synchronize()
        self.session.check_errors()
        host = {layer: [x.cpu() for x in ring] for layer, ring in self._rings.items()}
        log = self.session._log
        for position, histories in self._steps:
            slot, total = position % self.record_steps, position + 1
            for layer in sorted(histories):
                count, raw, valid = (x[slot] for x in host[layer])
                log.pending.append(dict(layer=layer, history=histories[layer], total=total,
                                        prefix=self.session.prefix_lengths[layer], unique=count, raw=raw,
                                        buckets=(valid > 0).sum(1)))
        self._steps = []

    def _prepare(self, total):
        """Lazy builds and updates for a step that ends with `total` tokens;
        True when any layer's history moved (the captured step is stale)."""
        s, moved = self.session, False
        for layer in s.modules:
            K = self.cache.layers[layer].keys[0]
            if layer not in s.ops:
                s._index(layer, K, total)
                moved = True
            if s.ops[layer].catch_up(K, total, s.update_interval):
                moved = True
        return moved

    def _forward(self):
        torch.remainder(self.pos.reshape(1), self.record_steps, out=self._slot)
        out = self.session.model(self.ids, position_ids=self.pos, attention_mask={"full_attention": None},
                                 past_key_values=self.cache, use_cache=True, logits_to_keep=1)
        return out.logits

    def _capture(self):
        # the replaced graph stays alive until the new one is captured into its pool
        old = self.graph
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=old.pool() if old is not None else None):
            self.logits = self._forward()
        self.graph, self.stale = graph, False

    @torch.no_grad()
    def __call__(self, ids):
        if self.position is None:  # the first step follows the prefill
            lengths = {self.session.prefix_lengths.get(layer) for layer in self.session.modules}
            if len(lengths) != 1 or None in lengths:
                raise RuntimeError("prefill every layer through the model before decoding")
            self.position = lengths.pop()
        if self.position >= self.max_length:
            raise ValueError("the static cache is full")
        self.session.check_errors()  # a give-up of an earlier replay surfaces here
        if self._prepare(self.position + 1):
            self.stale = True
        self.ids.copy_(ids.reshape(1, 1))
        self.pos.fill_(self.position)
        if not self.use_graph or self.eager_steps == 0:
            # eager: always without a graph, and once before the first capture
            # (library handles and workspaces are created outside the capture)
            logits = self._forward()
            self.eager_steps += 1
        else:
            if self.stale:
                self._capture()
            self.graph.replay()
            logits = self.logits
        self._steps.append((self.position, {layer: op.history for layer, op in self.session.ops.items()}))
        if len(self._steps) == self.record_steps:
            self.flush_records()
        self.position += 1
        return logits
