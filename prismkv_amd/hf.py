"""Hugging Face attention backend for unpadded, batch-one causal decoding
through the MI355X routed-decode path -- the native counterpart of
src/prismkv/hf_reference.py:65-240 (`HFReference`).

Prefill runs the model's own attention (SDPA or eager), as in the reference.
At a layer's first decode step its 8 KV groups are indexed on the device
from the prefix keys (`Native8B.build_index`, the reference's lazy
`build_index`, hf_reference.py:196-198); every decode step then indexes the
complete old tail blocks (`catch_up`, the update loop of :205-211) and runs
the single-launch decode (route, union, attention) for all 8 groups of the
layer at once.  The current token and the un-indexed tail are attended
densely, exactly as in the reference.

Native specialisation (rejected with NotImplementedError otherwise): Qwen3
attention with 8 KV heads x 4 query heads, head_dim 128, bf16 activations,
16 selected buckets (per query for router "q_activation", which routes,
unions up to 64 buckets and attends in four launches per layer).  `unique_cap` maps to
`Native8B.unique_cap`; mode "all_read" (the dense control) runs the model's
own attention over the whole cache.

The per-(layer, group) records of the reference (history, unique, raw,
buckets, tail, routing_policy) are kept as device tensors and read back
when `records` is first accessed after a step, so decoding does not
synchronise.

`DecodeGraph` (no reference counterpart; the role of the SM90 runner's
captured step, kernels/cuda_sm90/single.py:211-233) decodes from a
transformers `StaticCache`: the model's whole one-token forward, with every
layer's single-launch decode reading its tail length from the device, is
captured once in a HIP graph and replayed token after token; the lazy
builds and the update policy run eagerly between replays, and the step is
recaptured whenever a layer's history moves.
"""
from __future__ import annotations

import importlib
import math
from contextlib import contextmanager

import torch

from .native8b import DIM, GROUPS, HEADS, MAX_BLOCK, Native8B
from .weights import Encoder, layer_tables  # noqa: F401  (Encoder re-exported: reference name)

BACKEND = "prismkv_native"
BACKEND_EAGER = "prismkv_native_eager"


def _dispatch(module, q, k, v, attention_mask, **kwargs):
    session = getattr(module, "_prismkv_session", None)
    if session is None:
        raise RuntimeError("PrismKV backend selected without an attached session")
    return session.forward(module, q, k, v, attention_mask, **kwargs)


class HFNative:
    """Stateful all-group adapter; one session per model, one request at a
    time (same constructor arguments, methods and checks as the reference
    adapter).  `capacity_step` is the token granularity by which a layer's
    index capacity grows as the request gets longer."""

    def __init__(self, model, encoders, *, mode="sparse", router="moments", selected_buckets=16, unique_cap=None,
                 update_interval=4096, detailed_records=False, capacity_step=8192, library=None):
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
        self.model, self.encoders = model, encoders
        self.mode, self.router = mode, router
        self.selected_buckets, self.unique_cap = selected_buckets, unique_cap
        self.update_interval, self.force_prefill = update_interval, False
        self.detailed_records = detailed_records
        self.capacity_step, self.library = int(capacity_step), library
        self.modules, self.original, self.configs = {}, {}, {}
        expected = set()
        for module in model.modules():
            if type(module).__name__ not in ("Qwen3Attention", "Qwen3_5Attention"):
                continue
            if hasattr(module, "_prismkv_session"):
                raise ValueError("model already has a reference session")
            layer = module.layer_idx
            if layer in self.modules:
                raise ValueError("duplicate attention-layer IDs")
            cfg = module.config
            expected.update((layer, g) for g in range(cfg.num_key_value_heads))
            self.modules[layer] = module
            impl = cfg._attn_implementation
            if impl not in ("sdpa", "eager"):
                raise ValueError("reference adapter is validated for SDPA/eager prefill only")
            namespace = vars(importlib.import_module(type(module).__module__))
            self.original[layer] = (namespace["eager_attention_forward"] if impl == "eager"
                                    else namespace["ALL_ATTENTION_FUNCTIONS"][impl])
            self.configs[id(cfg)] = (cfg, impl)
        if not self.modules or set(encoders) != expected:
            raise ValueError(f"provide exactly all standard-attention KV encoders; missing={expected - set(encoders)}, "
                             f"extra={set(encoders) - expected}")
        from transformers import AttentionInterface, AttentionMaskInterface
        from transformers.masking_utils import eager_mask, sdpa_mask
        AttentionInterface.register(BACKEND, _dispatch)
        AttentionMaskInterface.register(BACKEND, sdpa_mask)
        # eager prefill needs an explicit causal mask (SDPA may elide it)
        AttentionInterface.register(BACKEND_EAGER, _dispatch)
        AttentionMaskInterface.register(BACKEND_EAGER, eager_mask)
        for module in self.modules.values():
            module._prismkv_session = self
        for cfg, old in self.configs.values():
            cfg._attn_implementation = BACKEND_EAGER if old == "eager" else BACKEND
        self._tables = {}  # layer -> encoder tables on the model's device
        self._static = None  # the DecodeGraph driving a static cache, if any
        self.begin_request()

    # ------------------------------------------------------------ lifecycle

    def begin_request(self):
        self.prefix_lengths, self.ops = {}, {}
        self._records, self._pending = [], []

    @contextmanager
    def prefill(self):
        """Explicitly mark chunked prefill, including one-token chunks."""
        previous = self.force_prefill
        self.force_prefill = True
        try:
            yield self
        finally:
            self.force_prefill = previous

    def close(self):
        for module in self.modules.values():
            if getattr(module, "_prismkv_session", None) is self:
                del module._prismkv_session
        for cfg, impl in self.configs.values():
            cfg._attn_implementation = impl
        self.ops.clear()

    def generate(self, *args, **kwargs):
        """Reset for a new model.generate call/cache."""
        if kwargs.get("past_key_values") is not None:
            raise ValueError("use manual model calls and session state for an existing cache")
        self.begin_request()
        return self.model.generate(*args, **kwargs)

    @property
    def records(self):
        """Per-(layer, group) decode records in the reference's fields."""
        if self._pending:
            torch.cuda.synchronize()
            self.check_errors()
            for layer, history, total, count, raw, buckets, prefix in self._pending:
                count, raw, buckets = count.tolist(), raw.tolist(), buckets.tolist()
                for g in range(GROUPS):
                    rec = dict(layer=layer, group=g, history=history, unique=count[g], raw=raw[g],
                               buckets=buckets[g], tail=total - history, routing_policy=self.mode)
                    if self.detailed_records:
                        rec.update(initial_history=prefix)
                    self._records.append(rec)
            self._pending = []
        return self._records

    def check_errors(self):
        """RuntimeError if a bounded wait of any layer's launches gave up
        (reads host-mapped words; no synchronisation)."""
        for op in self.ops.values():
            op.check_errors()

    # ------------------------------------------------------------ forward

    def _op(self, layer, K, total):
        op = self.ops.get(layer)
        if op is None:
            h = self.prefix_lengths[layer]
            if layer not in self._tables:
                self._tables[layer] = layer_tables(self.encoders, layer, GROUPS, K.device)
            W, b, scale, key_mean = self._tables[layer]
            op = Native8B.from_keys(K, h, W, b, scale, key_mean, self.library,
                                    capacity=self._capacity(total), unique_cap=self.unique_cap)
            if self.router == "q_activation":  # the same SAEs encode the queries (hf_reference.py:213-215)
                op.set_query_encoders(W, b, [float(self.encoders[(layer, g)].query_scale) for g in range(GROUPS)])
                op.router = "q_activation"
            self.ops[layer] = op
        if total > op.capacity:
            op.grow(self._capacity(total))
        return op

    def _capacity(self, total):
        if self._static is not None:  # a static cache never outgrows its buffers
            return self._static.max_length
        step = max(self.capacity_step, self.update_interval)
        return (total // step + 1) * step

    @torch.no_grad()
    def forward(self, module, q, k, v, attention_mask, **kwargs):
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
        layer, total, steps = module.layer_idx, k.shape[-2], q.shape[-2]
        if self._static is not None:
            return self._forward_static(module, q, k, v, attention_mask, **kwargs)
        if attention_mask is not None:
            if attention_mask.ndim != 4:
                raise NotImplementedError("padding/arbitrary attention masks are unsupported")
            last = attention_mask[..., -1, :total]
            invalid = ~last if last.dtype == torch.bool else last != 0
            if bool(invalid.any()):
                raise NotImplementedError("padding/arbitrary attention masks are unsupported")
        if self.force_prefill or layer not in self.prefix_lengths or steps > 1:
            self.prefix_lengths[layer] = total
            self.ops.pop(layer, None)
            if attention_mask is None and 1 < steps < total:
                # a cached chunk: supply the offset causal mask ourselves
                positions = torch.arange(total - steps, total, device=q.device)
                visible = torch.arange(total, device=q.device)[None] <= positions[:, None]
                attention_mask = torch.zeros((1, 1, steps, total), device=q.device, dtype=q.dtype)
                attention_mask.masked_fill_(~visible[None, None], -torch.inf)
            return self.original[layer](module, q, k, v, attention_mask, **kwargs)
        if steps != 1:
            raise NotImplementedError("decode reference is one token per forward")
        groups, queries = k.shape[1], q.shape[1]
        if queries % groups:
            raise ValueError("Q heads must form equal-sized KV groups")
        if groups != GROUPS or queries != GROUPS * HEADS or d != DIM or q.dtype != torch.bfloat16:
            raise NotImplementedError("the native path decodes 8 KV groups x 4 query heads, d=128, in bf16")
        prefix = self.prefix_lengths[layer]
        if self.mode == "all_read":
            self._pending.append((layer, prefix, total, torch.full((GROUPS,), prefix), torch.full((GROUPS,), prefix),
                                  torch.zeros(GROUPS, dtype=torch.long), prefix))
            return self.original[layer](module, q, k, v, attention_mask, **kwargs)
        K, V = k[0], v[0]
        if K.stride(-1) != 1 or K.stride(-2) != d:
            K, V = K.contiguous(), V.contiguous()
        op = self._op(layer, K, total)
        op.catch_up(K, total, self.update_interval)
        out = op(q[0, :, 0].reshape(GROUPS, HEADS, DIM).contiguous(), K, V)
        self._pending.append((layer, op.history, total, op.count.clone(), op.raw.clone(),
                              (op.valid > 0).sum(1), prefix))
        return out.reshape(1, 1, queries, d), None

    def _forward_static(self, module, q, k, v, attention_mask, **kwargs):
        """forward() over a StaticCache: K/V are the whole preallocated buffers
        and the positions come from `position_ids`.  Prefill (eager) runs the
        model's own attention under an explicit causal mask; a decode step
        launches the layer's single-launch decode with the tail length
        computed on the device, so it can be captured and replayed."""
        layer, steps, d = module.layer_idx, q.shape[-2], q.shape[-1]
        pos = kwargs.get("position_ids")
        if pos is None:
            raise ValueError("a static-cache forward passes position_ids")
        pos = pos.reshape(-1)
        if self.force_prefill or layer not in self.prefix_lengths or steps > 1:
            if q.is_cuda and torch.cuda.is_current_stream_capturing():
                raise RuntimeError("prefill cannot be captured")
            self.prefix_lengths[layer] = int(pos[-1]) + 1
            self.ops.pop(layer, None)
            if attention_mask is None:  # key j is visible to the query at position p iff j <= p
                visible = torch.arange(k.shape[-2], device=q.device)[None] <= pos.to(q.device)[:, None]
                attention_mask = torch.zeros((1, 1, steps, k.shape[-2]), device=q.device, dtype=q.dtype)
                attention_mask.masked_fill_(~visible[None, None], -torch.inf)
            return self.original[layer](module, q, k, v, attention_mask, **kwargs)
        if steps != 1:
            raise NotImplementedError("decode reference is one token per forward")
        groups, queries = k.shape[1], q.shape[1]
        if groups != GROUPS or queries != GROUPS * HEADS or d != DIM or q.dtype != torch.bfloat16:
            raise NotImplementedError("the native path decodes 8 KV groups x 4 query heads, d=128, in bf16")
        op = self.ops.get(layer)
        if op is None:
            raise RuntimeError("static-cache decode steps run through DecodeGraph")
        tail = (pos[-1:] + 1 - op.history).to(torch.int32)
        out = op(q[0, :, 0].reshape(GROUPS, HEADS, DIM).contiguous(), k[0], v[0], tail=tail)
        return out.reshape(1, 1, queries, d), None


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
    layer's single-launch decode (tail length = position + 1 - history,
    computed on the device).  With graph=False every step runs eagerly
    through the same code.  Sparse mode, the moments router and no unique cap
    only (the single-launch decode); records are not kept."""

    def __init__(self, session, cache, *, graph=True):
        if session.mode != "sparse" or session.router != "moments" or session.unique_cap is not None:
            raise NotImplementedError("DecodeGraph drives the single-launch decode: sparse mode, moments router, "
                                      "no unique cap")
        if session._static is not None:
            raise ValueError("the session already drives a static cache")
        device = next(session.model.parameters()).device
        self.session, self.cache, self.position = session, cache, None
        self.max_length = int(cache.max_cache_len)
        self.use_graph = bool(graph)
        self.ids = torch.zeros((1, 1), dtype=torch.long, device=device)
        self.pos = torch.zeros((1, 1), dtype=torch.long, device=device)
        self.graph, self.logits, self.stale = None, None, True
        self.eager_steps = 0
        session._static = self

    def close(self):
        if self.session._static is self:
            self.session._static = None
        self.graph = self.logits = None

    def _layer_keys(self, layer):
        keys = self.cache.layers[layer].keys
        return keys[0]

    def _prepare(self, total):
        """Lazy builds and updates for a step that ends with `total` tokens;
        True when any layer's history moved (the captured step is stale)."""
        s, moved = self.session, False
        for layer in s.modules:
            K = self._layer_keys(layer)
            if layer not in s.ops:
                s._op(layer, K, total)
                moved = True
            op = s.ops[layer]
            if op.catch_up(K, total, s.update_interval):
                moved = True
        return moved

    def _forward(self):
        out = self.session.model(self.ids, position_ids=self.pos, attention_mask={"full_attention": None},
                                 past_key_values=self.cache, use_cache=True, logits_to_keep=1)
        return out.logits

    @torch.no_grad()
    def __call__(self, ids):
        if self.position is None:  # the first step follows the prefill
            lengths = set(self.session.prefix_lengths.get(layer) for layer in self.session.modules)
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
                # the replaced graph stays alive until the new one is captured
                # into its memory pool
                old = self.graph
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, pool=old.pool() if old is not None else None):
                    self.logits = self._forward()
                self.graph, self.stale = graph, False
                del old
            self.graph.replay()
            logits = self.logits
        self.position += 1
        return logits

