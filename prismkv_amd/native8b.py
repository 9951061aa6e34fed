"""MI355X binding of PrismKV's native 8B decode path -- drop-in for
`prismkv.native8b` (src/prismkv/native8b.py).

Same class and method names, keyword arguments, attribute names, dtypes and
shapes as the reference binding:

* ``Native8B(indices, library)`` builds the device tables once per prefill /
  index rebuild (src/prismkv/native8b.py:35-74);
* ``.route(q)`` runs stage 1 (bucket routing) and stage 2 (bitmap union and
  compaction) and leaves ``features``, ``valid``, ``raw``, ``ids``, ``count``
  on the device (src/prismkv/native8b.py:82-89);
* ``.attention(q, k, v, *, splits=64, schedule=0)`` runs stage 3 and returns
  the preallocated ``out`` buffer, overwritten by the next call
  (src/prismkv/native8b.py:91-102);
* ``__call__`` = route + attention; ``buffer_bytes()`` lists live buffers;
* ``unique_cap`` (constructor keyword or attribute, default None) applies the
  strict unique-ID budget of ``select_buckets`` (src/prismkv/core.py:149-163):
  ranked buckets that would push the union past floor(history * unique_cap)
  tokens are skipped, and ``features`` / ``valid`` / ``raw`` list the kept
  buckets in rank order;
* ``append(k, block)`` is the reference's ``append_index``
  (src/prismkv/core.py:186-201) for all 8 groups on the device tables in
  place (after ``set_encoders``); ``catch_up`` is the update loop of
  src/prismkv/hf_reference.py:209-211; ``export_indices()`` reads the tables
  back as ``FeatureIndex`` objects.

All validation happens on the host before anything is enqueued (ValueError
for shapes/dtypes/devices/strides, RuntimeError for a nonzero launch code).
Every inter-workgroup wait of the kernels is bounded: a wait that gives up
marks a host-mapped error word of the instance, which the next route /
attention / call (and `check_errors`, `decode_errors`) reads without
synchronising and turns into a RuntimeError after resetting the
workspaces.
route/attention allocate nothing and never synchronise, so they can be
captured into a HIP graph.  Instance buffers are shared state: use one
instance per stream.  There is no CPU fallback: without the HIP library the
constructor raises.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from .build import compile_hip  # noqa: F401  (re-exported: reference name compile_ppu)

GROUPS, HEADS, DIM, FEATURES, TOPK = 8, 4, 128, 3000, 16
# Largest history the single-launch decode serves (256 workgroups per group
# of 2048 tokens each); longer histories take route + attention.
FUSED_MAX_HISTORY = 524288
# Largest block one `append` indexes (the reference's update interval is 4096,
# src/prismkv/hf_reference.py:75).
MAX_BLOCK = 4096
# Largest history one device index build covers (flat activation indices
# history * 3000 stay below 2^32).
MAX_BUILD = 1 << 20
# Workspace budget of a build: groups are indexed in batches whose dense
# activations (history x 3000 fp32 per group) fit in it.
BUILD_WORK_LIMIT = 8 << 30
# Workgroups per KV group of the sparse-attention launch (each 8 waves; one
# per CU at 8 groups x 32 = 256): the partition the kernel is tuned for.
ATTEND_SPLITS = 32
CHUNK = 32
CHUNKS = (FEATURES + CHUNK - 1) // CHUNK
# Codes of a workspace's error word (and the host-mapped word), as the kernels write them.
ERR_WAIT, ERR_IDS = 1, 2
ERROR_MESSAGES = {ERR_WAIT: "prismkv decode: a bounded inter-workgroup wait gave up",
                  ERR_IDS: "prismkv attention: an id outside [0, history) or a count outside [0, history] "
                           "reached the attention"}
PADDED = CHUNKS * CHUNK


@dataclass
class FeatureIndex:
    """Index state of one (layer, KV group), field-for-field the reference
    container (src/prismkv/core.py:62-73): original-token lists per bucket and
    count / mean / population diagonal variance of the original keys."""

    history: int
    center: torch.Tensor
    counts: torch.Tensor
    mean: torch.Tensor
    variance: torch.Tensor
    lists: list

    @property
    def memberships(self):
        return sum(len(x) for x in self.lists)


def set_spin_limit(limit: int, library=None) -> int:
    """Process-wide bound (in sleeps of 64 clocks) of every inter-workgroup
    wait of the kernels; returns the previous bound.  The default, 2^20, is
    tens of milliseconds; a smaller bound makes a wait give up (and report)
    sooner.  Launches read it when they are enqueued."""
    if int(limit) < 0:
        raise ValueError("the spin limit must be >= 0")
    return _lib.load(library).query("prismkv_set_spin_limit", int(limit))


def tile_moments(mean: torch.Tensor, variance: torch.Tensor) -> torch.Tensor:
    """[G,3000,128] mean and variance -> f32 [G,94,256,32] bucket tiles (k < 128 mean)."""
    g = mean.shape[0]
    rows = torch.cat((mean.float(), variance.float()), dim=-1)  # [G, F, 256]
    rows = torch.nn.functional.pad(rows, (0, 0, 0, PADDED - FEATURES))
    return rows.view(g, CHUNKS, CHUNK, 2 * DIM).permute(0, 1, 3, 2).contiguous()


def untile_moments(tiles: torch.Tensor):
    """Inverse of tile_moments -> (mean [G,3000,128], variance [G,3000,128])."""
    g = tiles.shape[0]
    rows = tiles.permute(0, 1, 3, 2).reshape(g, PADDED, 2 * DIM)[:, :FEATURES]
    return rows[..., :DIM], rows[..., DIM:]


def bitmap_row_words(capacity: int) -> int:
    """uint32 words per bucket row, rounded to 16 bytes for vector loads."""
    return ((capacity + 31) // 32 + 3) // 4 * 4


def _encoder_tables(saes, key_scales):
    """Stacked W_enc [8,3000,128], b_enc [8,3000] and the shared key_mean of 8 SAEs."""
    if len(saes) != GROUPS or len(key_scales) != GROUPS:
        raise ValueError("one SAE and key scale per KV group required")
    means = {int(s.key_mean) for s in saes}
    if len(means) != 1:
        raise ValueError("all groups must share one key_mean")
    W = torch.stack([torch.as_tensor(s.W_enc).detach() for s in saes])
    b = torch.stack([torch.as_tensor(s.b_enc).detach() for s in saes])
    return W, b, means.pop()


class Native8B:
    def __init__(self, indices, library=None, *, capacity=None, unique_cap=None):
        if len(indices) != GROUPS:
            raise ValueError("native specialization requires 8 KV groups")
        h = int(indices[0].history)
        device = indices[0].mean.device
        if device.type != "cuda":
            raise ValueError("native backend requires a device tensor")
        if any(x.history != h or tuple(x.mean.shape) != (FEATURES, DIM) for x in indices):
            raise ValueError("same history, F=3000, d=128 required")
        with torch.cuda.device(device):
            counts = torch.stack([torch.as_tensor(x.counts).to(device) for x in indices])
            width = max(max(x.memberships for x in indices), 1)
            # concatenate each group's lists where they live (host or device), then move once
            lists = [torch.cat([torch.as_tensor(l).reshape(-1) for l in x.lists]).to(device=device, dtype=torch.int32)
                     if x.memberships else torch.zeros(0, dtype=torch.int32, device=device) for x in indices]
            csr = torch.stack([torch.nn.functional.pad(x, (0, width - len(x))) for x in lists])
            offsets = torch.cat((torch.zeros(GROUPS, 1, dtype=torch.int64, device=device),
                                 counts.long().cumsum(1)), dim=1).int()
            self._setup(h, capacity, library, counts,
                        torch.stack([torch.as_tensor(x.mean).to(device) for x in indices]),
                        torch.stack([torch.as_tensor(x.variance).to(device) for x in indices]), csr, offsets,
                        torch.stack([torch.as_tensor(x.center).to(device) for x in indices]))
        self.unique_cap = unique_cap

    @classmethod
    def from_tables(cls, history, counts, mean, variance, csr_ids, offsets, library=None, *, capacity=None,
                    center=None, unique_cap=None):
        """Build from device tables directly: counts [8,3000], mean/variance
        [8,3000,128] f32, csr_ids i32 [8,C] (bucket f owns columns
        offsets[g,f] .. offsets[g,f+1]), offsets i32 [8,3001] and, for
        `append`, the indices' original centers [8,128]."""
        if counts.device.type != "cuda":
            raise ValueError("native backend requires a device tensor")
        if tuple(mean.shape) != (GROUPS, FEATURES, DIM) or mean.shape != variance.shape:
            raise ValueError("same history, F=3000, d=128 required")
        obj = cls.__new__(cls)
        with torch.cuda.device(counts.device):
            obj._setup(int(history), capacity, library, counts, mean, variance, csr_ids.int().contiguous(),
                       offsets.int().contiguous(), center)
        obj.unique_cap = unique_cap
        return obj

    @classmethod
    def from_keys(cls, k, history, W, b, key_scale, key_mean=8, library=None, *, center=None, capacity=None,
                  unique_cap=None, work_limit=BUILD_WORK_LIMIT, keep_activations=False):
        """build_index (src/prismkv/core.py:92-103) of all 8 groups on the
        device: K rows [0, history) of each group are encoded with its SAE
        (W [8,3000,128], b [8,3000], key_scale [8] > 0), the batch-wide
        positive Top-k with budget history * key_mean selects the
        memberships (flat-index tie rule, core.py:13-26), and every bucket's
        population mean and variance of the ORIGINAL keys fill the tables.
        The center is the mean of those K rows unless `center` [8,128] is
        given.  Returns a decode-ready instance whose encoders are set for
        `append`.  Groups are indexed in batches whose activations (history
        x 3000 fp32 each) fit in `work_limit` bytes; with keep_activations
        the last batch's activations stay readable (build_activations)."""
        if k.device.type != "cuda":
            raise ValueError("native backend requires a device tensor")
        history = int(history)
        if not 1 <= history <= MAX_BUILD:
            raise ValueError(f"history must be in [1, {MAX_BUILD}]")
        if k.dtype != torch.bfloat16 or k.dim() != 3 or k.shape[0] != GROUPS or k.shape[-1] != DIM:
            raise ValueError("BF16 K[8,total_length,128] required")
        if k.stride(-1) != 1 or k.stride(1) != DIM or k.shape[1] < history:
            raise ValueError("contiguous per-group K rows covering the history required")
        if (k.data_ptr() | (k.stride(0) * 2)) % 16:
            raise ValueError("K rows must be 16-byte aligned")
        obj = cls.__new__(cls)
        with torch.cuda.device(k.device):
            obj._allocate(history, capacity, library, k.device, center)
            obj.set_encoder_tables(W, b, key_scale, key_mean)
            flags = 0
            if obj.center is None:
                obj.center = torch.zeros(GROUPS, DIM, dtype=torch.float32, device=k.device)
                flags = 1  # the device computes the centers
            per_group = obj.lib.query("prismkv_build_work_bytes", 1, history)
            batch = max(1, min(GROUPS, int(work_limit) // per_group))
            work = torch.zeros(obj.lib.query("prismkv_build_work_bytes", batch, history), dtype=torch.uint8,
                               device=k.device)
            obj.lib.call("prismkv_build", k.data_ptr(), obj.W_enc.data_ptr(), obj.b_enc.data_ptr(),
                         obj.center.data_ptr(), obj.key_scale.data_ptr(), obj.bits.data_ptr(), obj.n.data_ptr(),
                         obj.moments.data_ptr(), work.data_ptr(), GROUPS, batch, history, obj.key_mean, flags,
                         k.stride(0), obj.row_words, _lib.nbytes(work), stream=obj._stream())
            obj.build_work = work if keep_activations else None
            obj.build_batch = batch
        obj.unique_cap = unique_cap
        return obj

    @classmethod
    def build_index(cls, k, saes, key_scales, history=None, library=None, **kwargs):
        """from_keys with the reference's encoder objects: `saes[g]` has
        W_enc [3000,128], b_enc [3000] and key_mean (SharedSAE,
        src/prismkv/core.py:29-48); history defaults to all rows of k."""
        W, b, key_mean = _encoder_tables(saes, key_scales)
        return cls.from_keys(k, k.shape[1] if history is None else history, W, b, key_scales, key_mean, library,
                             **kwargs)

    def build_activations(self):
        """Dense activations relu(x W^T + b) [batch, history, 3000] of the
        last group batch of from_keys(keep_activations=True): groups
        8 - batch .. 7."""
        if getattr(self, "build_work", None) is None:
            raise ValueError("build with keep_activations=True first")
        n = self.build_batch * self.history * FEATURES
        at = self.lib.query("prismkv_update_act_offset", self.build_batch)
        return self.build_work[at:at + 4 * n].view(torch.float32).view(self.build_batch, self.history, FEATURES)

    def _setup(self, h, capacity, library, counts, mean, variance, csr, offsets, center=None):
        if csr.numel() and (int(csr.max()) >= h or int(csr.min()) < 0):
            raise ValueError("bucket lists must address tokens in [0, history)")
        if offsets.shape != (GROUPS, FEATURES + 1) or int(offsets[:, -1].max()) > csr.shape[1]:
            raise ValueError("offsets must be [8,3001] within the list width")
        device = counts.device
        self._allocate(h, capacity, library, device, center)
        self.n[:, :FEATURES] = counts.int()
        self.moments.copy_(tile_moments(mean, variance))
        self.lib.call("prismkv_build_bits", csr.data_ptr(), offsets.data_ptr(), self.bits.data_ptr(), GROUPS,
                      csr.shape[1], self.row_words, stream=self._stream())
        # Temporary CSR storage may be freed after this build barrier.
        torch.cuda.synchronize(device)

    def _allocate(self, h, capacity, library, device, center=None):
        """Zeroed tables and buffers for history h (ids and bitmap columns for `capacity`)."""
        capacity = h if capacity is None else int(capacity)
        if capacity < h or h < 1:
            raise ValueError("history must be >= 1 and capacity >= history")
        self.history = h
        self.capacity = capacity
        self.lib = _lib.load(library)
        if self.lib.missing:
            raise RuntimeError(f"{self.lib.path.name} lacks entry points {self.lib.missing}; rebuild it")
        self.n = torch.zeros(GROUPS, PADDED, dtype=torch.int32, device=device)
        self.moments = torch.zeros(GROUPS, CHUNKS, 2 * DIM, CHUNK, dtype=torch.float32, device=device)
        self.features = torch.zeros(GROUPS, TOPK, dtype=torch.int64, device=device)
        self.valid = torch.zeros(GROUPS, TOPK, device=device)
        self.raw = torch.zeros(GROUPS, dtype=torch.int32, device=device)
        self.ids = torch.zeros(GROUPS, self.capacity, dtype=torch.int32, device=device)
        self.count = torch.zeros(GROUPS, dtype=torch.int32, device=device)
        self.row_words = bitmap_row_words(self.capacity)
        self.bits = torch.zeros(GROUPS, FEATURES, self.row_words, dtype=torch.int32, device=device)
        self.union_work = torch.zeros(self.lib.query("prismkv_union_work_bytes", GROUPS, self.capacity),
                                      dtype=torch.uint8, device=device)
        self.state = torch.zeros(self.lib.query("prismkv_attend_work_bytes", GROUPS, ATTEND_SPLITS),
                                 dtype=torch.uint8, device=device)
        self.decode_work = torch.zeros(self.lib.query("prismkv_decode_work_bytes", GROUPS, self.capacity),
                                       dtype=torch.uint8, device=device)
        # host-mapped error word the kernels mark when a bounded wait gives up
        self._err_host = torch.zeros(4, dtype=torch.int32, pin_memory=True)
        self._err_device_address = self.lib.query("prismkv_mapped_pointer", self._err_host.data_ptr())
        if not self._err_device_address:
            raise RuntimeError("prismkv_mapped_pointer: the pinned error word is not device-accessible")
        self._attach_error_word()
        self.out = torch.zeros(GROUPS, HEADS, DIM, dtype=torch.bfloat16, device=device)
        self.center = None if center is None else center.to(device=device, dtype=torch.float32).reshape(
            GROUPS, DIM).contiguous()
        # encoder tables and block workspace of `append`, set by set_encoders
        self.W_enc = self.b_enc = self.key_scale = self.update_work = None
        self.W_query = self.b_query = self.query_scale = self.qact_work = None
        self.key_mean = 0
        self.update_block = 0

    def _stream(self):
        return torch.cuda.current_stream().cuda_stream

    def _attach_error_word(self):
        """Writes the host-mapped error word's device address into the
        host-word slot (bytes 8-15) of the workspaces whose kernels wait."""
        for work in (self.decode_work, self.union_work, self.state):
            work[8:16].view(torch.int64).fill_(self._err_device_address)

    def check_errors(self):
        """Raise RuntimeError if an earlier launch reported an error: a
        bounded inter-workgroup wait gave up, or the attention found an id
        outside [0, history) in `ids` (or a count outside [0, history]) and
        read it clamped.  Either way the results of the launches since the
        last check are invalid.  Reads the host-mapped error word, so it
        neither synchronises nor sees launches that have not run yet; on an
        error the device is synchronised, every workspace is zeroed (a late
        workgroup may have left published words behind) and the error words
        are cleared before raising."""
        code = int(self._err_host[0])
        if code == 0:
            return
        self.reset_workspaces()
        raise RuntimeError(ERROR_MESSAGES.get(code, ERROR_MESSAGES[ERR_WAIT]) + "; the results of the launches "
                           "since the last check are invalid (the workspaces have been reset)")

    def reset_workspaces(self):
        """Zero the decode, union and attention workspaces and the error
        words (after synchronising the device)."""
        torch.cuda.synchronize(self.out.device)
        for work in (self.decode_work, self.union_work, self.state):
            work.zero_()
        self._err_host.zero_()
        self._attach_error_word()
        torch.cuda.synchronize(self.out.device)

    @property
    def unique_cap(self):
        return self.__dict__.get("_unique_cap")

    @unique_cap.setter
    def unique_cap(self, cap):
        # same check and message as src/prismkv/core.py:149-150
        if cap is not None and not 0 <= cap <= 1:
            raise ValueError("unique_cap must be a fraction in [0,1]")
        self.__dict__["_unique_cap"] = cap

    def route(self, q):
        """Stages 1-2: features / valid / raw and the union's ids / count.
        With the moments router, no unique cap and a history the fused
        decode serves, ONE launch (prismkv_route_union: the decode's
        selection, union and id phases without the attention)."""
        self.check_errors()
        if self.router == "moments" and self.unique_cap is None and self.history <= FUSED_MAX_HISTORY:
            if tuple(q.shape) != (GROUPS, HEADS, DIM) or q.dtype != torch.bfloat16 or not q.is_contiguous():
                raise ValueError("contiguous BF16 Q[8,4,128] required")
            if q.device != self.out.device:
                raise ValueError("Q must live on the index device")
            self.lib.call("prismkv_route_union", q.data_ptr(), self.moments.data_ptr(), self.n.data_ptr(),
                          self.bits.data_ptr(), self.decode_work.data_ptr(), self.features.data_ptr(),
                          self.valid.data_ptr(), self.raw.data_ptr(), self.ids.data_ptr(), self.count.data_ptr(),
                          GROUPS, self.history, self.capacity, self.row_words, self.capacity,
                          _lib.nbytes(self.decode_work), stream=self._stream())
            return
        width = self._select(q)
        self.lib.call("prismkv_union_n", self.bits.data_ptr(), self.features.data_ptr(), self.valid.data_ptr(),
                      self.union_work.data_ptr(), self.ids.data_ptr(), self.count.data_ptr(), GROUPS, self.history,
                      self.row_words, self.capacity, width, _lib.nbytes(self.union_work), stream=self._stream())

    def _select(self, q):
        """Stage 1 and the optional strict unique cap: features / valid / raw.
        Returns the selection width (16, or 64 for the q_activation router)."""
        if tuple(q.shape) != (GROUPS, HEADS, DIM) or q.dtype != torch.bfloat16 or not q.is_contiguous():
            raise ValueError("contiguous BF16 Q[8,4,128] required")
        if q.device != self.out.device:
            raise ValueError("Q must live on the index device")
        s = self._stream()
        if self.router == "q_activation":
            self.lib.call("prismkv_route_qact", q.data_ptr(), self.W_query.data_ptr(), self.b_query.data_ptr(),
                          self.query_scale.data_ptr(), self.n.data_ptr(), self.qact_work.data_ptr(),
                          self.features.data_ptr(), self.valid.data_ptr(), self.raw.data_ptr(), 0, GROUPS,
                          _lib.nbytes(self.qact_work), stream=s)
        else:
            # one launch: the selection phases of the decode, on its workspace
            self.lib.call("prismkv_route_single", q.data_ptr(), self.moments.data_ptr(), self.n.data_ptr(),
                          self.decode_work.data_ptr(), self.features.data_ptr(), self.valid.data_ptr(),
                          self.raw.data_ptr(), GROUPS, _lib.nbytes(self.decode_work), stream=s)
        width = self.features.shape[1]
        if self.unique_cap is not None:
            self.lib.call("prismkv_select_cap_n", self.bits.data_ptr(), self.n.data_ptr(), self.features.data_ptr(),
                          self.valid.data_ptr(), self.raw.data_ptr(), GROUPS, self.history, self._cap_limit(),
                          self.row_words, width, stream=s)
        return width

    def _cap_limit(self):
        """The strict unique cap's limit, floor(history * unique_cap)
        (src/prismkv/core.py:155)."""
        return math.floor(self.history * self.unique_cap)

    @property
    def router(self):
        return self.__dict__.get("_router", "moments")

    @router.setter
    def router(self, router):
        """"moments" (the native path, one launch per layer) or "q_activation"
        (src/prismkv/core.py:131-139: route + union of up to 64 buckets, then
        attention; needs set_query_encoders).  features / valid are [8,16]
        for moments and [8,64] for q_activation."""
        if router not in ("moments", "q_activation"):
            raise ValueError("unsupported router/bucket count")
        if router == "q_activation" and getattr(self, "W_query", None) is None:
            raise ValueError("q_activation requires SAE and saved positive query scale")
        width = TOPK if router == "moments" else 4 * TOPK
        if self.features.shape[1] != width:
            device = self.out.device
            self.features = torch.zeros(GROUPS, width, dtype=torch.int64, device=device)
            self.valid = torch.zeros(GROUPS, width, device=device)
        self.__dict__["_router"] = router

    def set_query_encoders(self, W, b, query_scale):
        """Encoders of the queries for router "q_activation": W [8,3000,128],
        b [8,3000] (the groups' SAEs) and query_scale [8] > 0."""
        device = self.out.device
        W = torch.as_tensor(W).to(device=device, dtype=torch.float32).contiguous()
        b = torch.as_tensor(b).to(device=device, dtype=torch.float32).contiguous()
        scale = torch.as_tensor(query_scale, dtype=torch.float32).reshape(-1).to(device)
        if tuple(W.shape) != (GROUPS, FEATURES, DIM) or tuple(b.shape) != (GROUPS, FEATURES):
            raise ValueError("W_enc [8,3000,128] and b_enc [8,3000] required")
        if scale.numel() != GROUPS or not bool((scale > 0).all()):
            raise ValueError("q_activation requires SAE and saved positive query scale")
        self.W_query, self.b_query, self.query_scale = W, b, scale.contiguous()
        self.qact_work = torch.zeros(self.lib.query("prismkv_route_qact_work_bytes", GROUPS), dtype=torch.uint8,
                                     device=device)

    def _check_kv(self, q, k, v, splits, schedule):
        if not 1 <= splits <= 128 or schedule not in (0, 1, 2):
            raise ValueError("unsupported attention partition/schedule")
        if k.shape != v.shape or k.shape[0] != GROUPS or k.shape[-1] != DIM or k.shape[1] < self.history:
            raise ValueError("K/V[8,total_length,128] required")
        if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16 or k.stride(-1) != 1 or v.stride(-1) != 1:
            raise ValueError("BF16 KV with contiguous head dimension required")
        if k.stride(1) != DIM or v.stride(1) != DIM:
            raise ValueError("contiguous per-group KV rows required")
        if tuple(q.shape) != (GROUPS, HEADS, DIM) or q.dtype != torch.bfloat16 or not q.is_contiguous():
            raise ValueError("contiguous BF16 Q[8,4,128] required")
        if not (q.device == k.device == v.device == self.out.device):
            raise ValueError("Q/K/V must live on the index device")
        if (q.data_ptr() | k.data_ptr() | v.data_ptr() | (k.stride(0) * 2) | (v.stride(0) * 2)) % 16:
            raise ValueError("Q/K/V rows must be 16-byte aligned")

    def attention(self, q, k, v, *, splits=64, schedule=0):
        """Stage 3.  `splits` (1..128) and `schedule` (0, 1, 2) are validated and
        accepted for compatibility; the softmax is exact, so the partition does
        not change the result.  The launch is the fused decode's attention
        phases over the selection's ids (every S-th 16-row chunk of a group's
        rows per workgroup, contiguous shares of a list longer than 512 S);
        a wait that gives up is reported at the next call."""
        self._check_kv(q, k, v, splits, schedule)
        self.check_errors()
        self.lib.call("prismkv_attend", q.data_ptr(), k.data_ptr(), v.data_ptr(), self.ids.data_ptr(),
                      self.count.data_ptr(), self.state.data_ptr(), self.out.data_ptr(), GROUPS, self.history,
                      k.shape[1] - self.history, k.stride(0), v.stride(0), self.capacity, ATTEND_SPLITS,
                      _lib.nbytes(self.state), stream=self._stream())
        return self.out

    def __call__(self, q, k, v, *, tail=None, **kwargs):
        """route + attention (src/prismkv/native8b.py:104-106) through the fused
        decode path: one launch, every output buffer (features, valid, raw,
        ids, count, out) written as by the two calls -- the selection and ids
        bit-identical, out within rounding of the separate attention kernel.
        With a unique cap the same launch runs the budgeted walk between the
        selection and the union (features / valid / raw then hold the kept
        buckets, compacted in rank order, as route() leaves them).

        `tail` (no reference counterpart): an int32 CUDA tensor of one element
        holding the tail length T, read by the kernel at launch instead of
        taking T = K rows - history from K's shape; K/V then only need rows
        for T up to their length (a static KV buffer).  A launch captured in a
        HIP graph is replayed with whatever the tensor holds, clamped to
        [0, K rows - history].  The moments router with histories up to
        FUSED_MAX_HISTORY (the single launch, with or without a cap)."""
        self._check_kv(q, k, v, kwargs.get("splits", 64), kwargs.get("schedule", 0))
        self.check_errors()
        if tail is not None:
            if self.history > FUSED_MAX_HISTORY or self.router != "moments":
                raise NotImplementedError("a device tail length needs the fused decode (history <= "
                                          "FUSED_MAX_HISTORY, moments router)")
            if (not isinstance(tail, torch.Tensor) or tail.dtype != torch.int32 or tail.numel() != 1
                    or tail.device != self.out.device):
                raise ValueError("tail must be a one-element int32 tensor on the index device")
            if self.unique_cap is not None:
                self.lib.call("prismkv_decode_capped_tail", q.data_ptr(), self.moments.data_ptr(),
                              self.n.data_ptr(), self.bits.data_ptr(), k.data_ptr(), v.data_ptr(),
                              self.decode_work.data_ptr(), self.features.data_ptr(), self.valid.data_ptr(),
                              self.raw.data_ptr(), self.ids.data_ptr(), self.count.data_ptr(), self.out.data_ptr(),
                              tail.data_ptr(), GROUPS, self.history, k.shape[1] - self.history, self.capacity,
                              self._cap_limit(), self.row_words, k.stride(0), v.stride(0), self.capacity,
                              _lib.nbytes(self.decode_work), stream=self._stream())
                return self.out
            self.lib.call("prismkv_decode_tail", q.data_ptr(), self.moments.data_ptr(), self.n.data_ptr(),
                          self.bits.data_ptr(), k.data_ptr(), v.data_ptr(), self.decode_work.data_ptr(),
                          self.features.data_ptr(), self.valid.data_ptr(), self.raw.data_ptr(), self.ids.data_ptr(),
                          self.count.data_ptr(), self.out.data_ptr(), tail.data_ptr(), GROUPS, self.history,
                          k.shape[1] - self.history, self.capacity, self.row_words, k.stride(0), v.stride(0),
                          self.capacity, _lib.nbytes(self.decode_work), stream=self._stream())
            return self.out
        if self.history > FUSED_MAX_HISTORY or self.router != "moments":
            # very long histories exceed one launch's group size; the q_activation
            # router selects up to 64 buckets
            self.route(q)
            return self.attention(q, k, v, **kwargs)
        if self.unique_cap is not None:
            # the budgeted walk runs between selection and union, on the same launch
            self.lib.call("prismkv_decode_capped", q.data_ptr(), self.moments.data_ptr(), self.n.data_ptr(),
                          self.bits.data_ptr(), k.data_ptr(), v.data_ptr(), self.decode_work.data_ptr(),
                          self.features.data_ptr(), self.valid.data_ptr(), self.raw.data_ptr(), self.ids.data_ptr(),
                          self.count.data_ptr(), self.out.data_ptr(), GROUPS, self.history,
                          k.shape[1] - self.history, self.capacity, self._cap_limit(), self.row_words, k.stride(0),
                          v.stride(0), self.capacity, _lib.nbytes(self.decode_work), stream=self._stream())
            return self.out
        self.lib.call("prismkv_decode", q.data_ptr(), self.moments.data_ptr(), self.n.data_ptr(), self.bits.data_ptr(),
                      k.data_ptr(), v.data_ptr(), self.decode_work.data_ptr(), self.features.data_ptr(),
                      self.valid.data_ptr(), self.raw.data_ptr(), self.ids.data_ptr(), self.count.data_ptr(),
                      self.out.data_ptr(), GROUPS, self.history, k.shape[1] - self.history, self.capacity,
                      self.row_words, k.stride(0), v.stride(0), self.capacity, _lib.nbytes(self.decode_work),
                      stream=self._stream())
        return self.out

    # ------------------------------------------------------------ stage 4

    def set_encoders(self, saes, key_scales):
        """Per-group encoders for `append`: `saes[g]` has W_enc [3000,128],
        b_enc [3000] and key_mean (SharedSAE, src/prismkv/core.py:29-48) and
        `key_scales[g]` > 0 is its key scale -- the reference's
        encoders[(layer, group)] bundle (src/prismkv/hf_reference.py:196-211)."""
        W, b, key_mean = _encoder_tables(saes, key_scales)
        self.set_encoder_tables(W, b, key_scales, key_mean)

    def set_encoder_tables(self, W, b, key_scale, key_mean):
        """Encoder tables directly: W [8,3000,128], b [8,3000], key_scale [8]
        (each > 0), key_mean in [1, 3000].  Copied to the device as f32."""
        device = self.out.device
        W = torch.as_tensor(W).to(device=device, dtype=torch.float32).contiguous()
        b = torch.as_tensor(b).to(device=device, dtype=torch.float32).contiguous()
        scale = torch.as_tensor(key_scale, dtype=torch.float32).reshape(-1).to(device)
        if tuple(W.shape) != (GROUPS, FEATURES, DIM) or tuple(b.shape) != (GROUPS, FEATURES):
            raise ValueError("W_enc [8,3000,128] and b_enc [8,3000] required")
        if scale.numel() != GROUPS or not bool((scale > 0).all()):
            raise ValueError("positive key_scale per group required")
        if not 1 <= int(key_mean) <= FEATURES:
            raise ValueError("invalid sparsity")
        self.W_enc, self.b_enc, self.key_scale, self.key_mean = W, b, scale.contiguous(), int(key_mean)

    def append(self, k, block):
        """append_index (src/prismkv/core.py:186-201) for all 8 groups: index
        K rows [history, history + block) with the encoders and the ORIGINAL
        centers, BatchTopK over the block only (budget block * key_mean),
        merge their moments into the tables and add their memberships; then
        history += block.  Enqueued on the current stream; the workspace is
        allocated on the first call with a larger block than before."""
        if self.W_enc is None:
            raise ValueError("set_encoders before append")
        if self.center is None:
            raise ValueError("the index centers are required to append")
        block = int(block)
        if not 1 <= block <= MAX_BLOCK:
            raise ValueError(f"block must be in [1, {MAX_BLOCK}]")
        if k.dtype != torch.bfloat16 or k.dim() != 3 or k.shape[0] != GROUPS or k.shape[-1] != DIM:
            raise ValueError("BF16 K[8,total_length,128] required")
        if k.stride(-1) != 1 or k.stride(1) != DIM or k.device != self.out.device:
            raise ValueError("contiguous per-group K rows on the index device required")
        if k.shape[1] < self.history + block:
            raise ValueError("K does not hold the block to index")
        if self.history + block > self.capacity:
            raise ValueError("capacity exceeded: rebuild with a larger capacity")
        if block > self.update_block:
            self.update_work = torch.zeros(self.lib.query("prismkv_update_work_bytes", GROUPS, block),
                                           dtype=torch.uint8, device=self.out.device)
            self.update_block = block
        self.lib.call("prismkv_update", k.data_ptr(), self.W_enc.data_ptr(), self.b_enc.data_ptr(),
                      self.center.data_ptr(), self.key_scale.data_ptr(), self.bits.data_ptr(), self.n.data_ptr(),
                      self.moments.data_ptr(), self.update_work.data_ptr(), GROUPS, self.history, block,
                      self.key_mean, k.stride(0), self.row_words, _lib.nbytes(self.update_work),
                      stream=self._stream())
        self.history += block

    def update_activations(self, block):
        """The last append's dense activations relu(x W^T + b) [8,block,3000]
        (a view of the workspace, valid until the next append)."""
        if self.update_work is None or not 1 <= block <= self.update_block:
            raise ValueError("no append with this block size")
        n = GROUPS * block * FEATURES
        at = self.lib.query("prismkv_update_act_offset", GROUPS)
        return self.update_work[at:at + 4 * n].view(torch.float32).view(GROUPS, block, FEATURES)

    def catch_up(self, k, total=None, update_interval=MAX_BLOCK):
        """Index complete old tail blocks while more than `update_interval`
        tokens follow the history (src/prismkv/hf_reference.py:209-211);
        returns the number of blocks appended."""
        total = k.shape[1] if total is None else int(total)
        blocks = 0
        while total - self.history > update_interval:
            self.append(k, update_interval)
            blocks += 1
        return blocks

    def grow(self, capacity):
        """Extend the id and bitmap capacity to `capacity` tokens, keeping
        every membership (bitmap columns are copied into wider rows; the
        workspaces are reallocated zeroed).  Enqueued on the current stream."""
        capacity = int(capacity)
        if capacity <= self.capacity:
            return
        device = self.out.device
        rw = bitmap_row_words(capacity)
        bits = torch.zeros(GROUPS, FEATURES, rw, dtype=torch.int32, device=device)
        bits[:, :, :self.row_words] = self.bits
        self.bits, self.row_words, self.capacity = bits, rw, capacity
        self.ids = torch.zeros(GROUPS, capacity, dtype=torch.int32, device=device)
        self.union_work = torch.zeros(self.lib.query("prismkv_union_work_bytes", GROUPS, capacity),
                                      dtype=torch.uint8, device=device)
        self.decode_work = torch.zeros(self.lib.query("prismkv_decode_work_bytes", GROUPS, capacity),
                                       dtype=torch.uint8, device=device)
        self._attach_error_word()

    def export_indices(self):
        """The device tables as 8 FeatureIndex objects (counts i64, mean and
        variance f32 [3000,128], centers on the device; per-bucket ascending
        token lists as host int64 tensors).  Synchronises; allocates."""
        mean, var = untile_moments(self.moments)
        h = self.history
        shifts = torch.arange(32, device=self.bits.device, dtype=torch.int32)
        out = []
        for g in range(GROUPS):
            words = self.bits[g, :, :(h + 31) // 32]
            flags = ((words.unsqueeze(-1) >> shifts) & 1).to(torch.bool).reshape(FEATURES, -1)[:, :h]
            f, t = flags.nonzero(as_tuple=True)
            per = torch.bincount(f, minlength=FEATURES).tolist()
            lists = list(torch.split(t.cpu(), per))
            center = None if self.center is None else self.center[g].clone()
            out.append(FeatureIndex(h, center, self.n[g, :FEATURES].long().clone(), mean[g].contiguous(),
                                    var[g].contiguous(), lists))
        return out

    def decode_errors(self):
        """Nonzero if a bounded inter-workgroup wait of any launch since the
        last reset gave up (the decode, union and attention workspaces'
        sticky error words and the host-mapped word); synchronises, raises
        nothing."""
        torch.cuda.synchronize(self.out.device)
        return (int(self.decode_work[:4].view(torch.int32).item()) | int(self.union_work[:4].view(torch.int32).item())
                | int(self.state[:4].view(torch.int32).item()) | int(self._err_host[0]))

    def buffer_bytes(self):
        """Live tensors owned here; excludes model/KV, caller indices and build temporaries."""
        return {name: x.numel() * x.element_size() for name, x in vars(self).items() if isinstance(x, torch.Tensor)}
