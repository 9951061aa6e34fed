"""CPU oracle for PrismKV's routed-decode path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithm on the CPU (C in
``prismkv_oracle.c``, numpy around it) so that tests, the smoke entry point and
the bench's CPU-baseline leg can check the HIP path.  The shipped package
``prismkv_amd`` never imports it.

Each wrapper names the reference file:line its C function follows.  Floating
point is carried in double precision and rounded once; orderings come with a
relative ``margin`` (smallest gap between neighbouring ranks) so a test can
separate a real disagreement from a rounding-order near-tie.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
SOURCE = HERE / "prismkv_oracle.c"

_lib = None


def build(force: bool = False) -> Path:
    """Compile the C oracle with gcc into oracle/liboracle.so."""
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < SOURCE.stat().st_mtime:
        tmp = LIB_PATH.with_suffix(".so.tmp")
        subprocess.run(["gcc", "-O2", "-std=c11", "-shared", "-fPIC", "-o", str(tmp), str(SOURCE), "-lm"],
                       check=True)
        os.replace(tmp, LIB_PATH)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F32 = ctypes.c_float
F64 = ctypes.c_double


def _declare(L):
    sig = {
        "orc_f32_to_bf16": ([F32], ctypes.c_uint16),
        "orc_positive_global_topk": ([P, I64, I64, P], I64),
        "orc_topk_margin": ([P, I64, I64], F64),
        "orc_sae_dense": ([P, I64, I32, P, P, I32, P], None),
        "orc_summarize": ([P, I32, P, P, I32, P, P, P], None),
        "orc_mean_rows": ([P, I64, I32, P], None),
        "orc_build_index": ([P, I64, I32, P, P, I32, I32, F32, P, P, P, P, P, P, P, P], I64),
        "orc_merge_moments": ([I32, I32, P, P, P, P, P, P, P, P, P], None),
        "orc_bucket_scores": ([P, I32, I32, P, P, P, I32, I32, I32, P, P, P, P], I32),
        "orc_qact_scores": ([P, I32, I32, P, P, I32, F32, P, I32, P, P, P], I32),
        "orc_norm_top": ([P, P, P, I32, I32, I32, P, P, P, P, P], I32),
        "orc_pack": ([P, I32, I32, P], None),
        "orc_select_buckets": ([P, I32, P, P, I64, F64, P, P, P, P, P], I64),
        "orc_build_bits": ([P, P, I32, I64, P], None),
        "orc_union_bits": ([P, I64, I64, P, P, I32, P], I64),
        "orc_attend": ([P, I32, I32, P, P, I64, I64, P, I64, I64, P], I32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- bf16 helpers

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns (uint16) to float32."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def rel_l2(actual, expected) -> float:
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-8))


# ---------------------------------------------------------------- CSR lists

def lists_to_csr(lists):
    counts = np.array([len(x) for x in lists], dtype=np.int64)
    offsets = np.zeros(len(lists) + 1, dtype=np.int64)
    np.cumsum(counts, out=offsets[1:])
    ids = np.concatenate([np.asarray(x, dtype=np.int64) for x in lists]) if len(lists) else np.zeros(0, np.int64)
    return offsets, ids


def csr_to_lists(offsets, ids):
    return [ids[offsets[f]:offsets[f + 1]] for f in range(len(offsets) - 1)]


# ---------------------------------------------------------------- stage 4

def positive_global_topk(a: np.ndarray, count: int) -> np.ndarray:
    """src/prismkv/core.py:13-26 (strict ascending, then ties ascending)."""
    if a.ndim != 2 or count < 0:
        raise ValueError("expected a matrix and nonnegative activation budget")
    flat = _c(a.reshape(-1), np.float32)
    out = np.empty(max(min(count, flat.size), 1), dtype=np.int64)
    n = lib().orc_positive_global_topk(_ptr(flat), flat.size, count, _ptr(out))
    return out[:n]


def topk_margin(a: np.ndarray, count: int) -> float:
    flat = _c(a.reshape(-1), np.float32)
    return lib().orc_topk_margin(_ptr(flat), flat.size, count)


def sae_dense(x: np.ndarray, W: np.ndarray, b: np.ndarray) -> np.ndarray:
    """src/prismkv/core.py:47-48: relu(x @ W^T + b), double accumulation."""
    x = _c(x, np.float32)
    W = _c(W, np.float32)
    b = _c(b, np.float32)
    N, d = x.shape
    F = W.shape[0]
    out = np.empty((N, F), dtype=np.float32)
    lib().orc_sae_dense(_ptr(x), N, d, _ptr(W), _ptr(b), F, _ptr(out))
    return out


def summarize(keys: np.ndarray, lists):
    """src/prismkv/core.py:76-89 -> (counts i64[F], mean f32[F,d], var f32[F,d])."""
    keys = _c(keys, np.float32)
    offsets, ids = lists_to_csr(lists)
    F, d = len(lists), keys.shape[1]
    counts = np.empty(F, np.int64)
    mean = np.empty((F, d), np.float32)
    var = np.empty((F, d), np.float32)
    lib().orc_summarize(_ptr(keys), d, _ptr(offsets), _ptr(_c(ids, np.int64)), F, _ptr(counts), _ptr(mean),
                        _ptr(var))
    return counts, mean, var


class Index:
    """Mirror of the reference FeatureIndex (src/prismkv/core.py:62-73), numpy-backed."""

    def __init__(self, history, center, counts, mean, variance, lists):
        self.history = int(history)
        self.center = np.asarray(center, np.float32)
        self.counts = np.asarray(counts, np.int64)
        self.mean = np.asarray(mean, np.float32)
        self.variance = np.asarray(variance, np.float32)
        self.lists = [np.asarray(x, np.int64) for x in lists]

    @property
    def memberships(self):
        return int(sum(len(x) for x in self.lists))


def build_index(keys, W, b, key_scale, key_mean=8, center=None, return_act=False):
    """src/prismkv/core.py:92-103 on the CPU (double-accumulated SAE encode)."""
    keys = _c(keys, np.float32)
    W = _c(W, np.float32)
    b = _c(b, np.float32)
    N, d = keys.shape
    F = W.shape[0]
    if N == 0 or not key_scale > 0:
        raise ValueError("nonempty [history,head_dim] keys and positive scale required")
    c_out = np.empty(d, np.float32)
    act = np.empty((N, F), np.float32)
    offsets = np.empty(F + 1, np.int64)
    ids = np.empty(max(N * key_mean, 1), np.int64)
    counts = np.empty(F, np.int64)
    mean = np.empty((F, d), np.float32)
    var = np.empty((F, d), np.float32)
    cin = None if center is None else _c(center, np.float32)
    n = lib().orc_build_index(_ptr(keys), N, d, _ptr(W), _ptr(b), F, key_mean, float(key_scale),
                              None if cin is None else _ptr(cin), _ptr(c_out), _ptr(act), _ptr(offsets),
                              _ptr(ids), _ptr(counts), _ptr(mean), _ptr(var))
    if n < 0:
        raise ValueError("invalid build_index arguments")
    index = Index(N, c_out, counts, mean, var, csr_to_lists(offsets, ids[:n]))
    return (index, act) if return_act else index


def merge_moments(ca, ma, va, cb, mb, vb):
    """src/prismkv/core.py:190-199 (Chan merge of two populations per bucket)."""
    F, d = ma.shape
    co = np.empty(F, np.int64)
    mo = np.empty((F, d), np.float32)
    vo = np.empty((F, d), np.float32)
    args = [_c(ca, np.int64), _c(ma, np.float32), _c(va, np.float32), _c(cb, np.int64), _c(mb, np.float32),
            _c(vb, np.float32)]
    lib().orc_merge_moments(F, d, *[_ptr(a) for a in args], _ptr(co), _ptr(mo), _ptr(vo))
    return co, mo, vo


def append_index(index: Index, new_keys, W, b, key_scale, key_mean=8, return_act=False):
    """src/prismkv/core.py:186-201: index the new block with the ORIGINAL center,
    BatchTopK over the block only, merge moments, append lists shifted by history."""
    nxt, act = build_index(new_keys, W, b, key_scale, key_mean, center=index.center, return_act=True)
    co, mo, vo = merge_moments(index.counts, index.mean, index.variance, nxt.counts, nxt.mean, nxt.variance)
    lists = [np.concatenate((old, new + index.history)) for old, new in zip(index.lists, nxt.lists)]
    out = Index(index.history + len(new_keys), index.center, co, mo, vo, lists)
    return (out, act) if return_act else out


# ---------------------------------------------------------------- stage 1

TERMS = {"count": 1, "mean": 2, "variance": 4}


def bucket_scores(q, counts, mean, var, topk=16, terms=("count", "mean", "variance")):
    """src/prismkv/core.py:106-130 (router="moments") -> (score f64[F], order i64[<=topk], margin, ties)."""
    q = _c(q, np.float32)
    Hq, d = q.shape
    counts = _c(counts, np.int64)
    F = counts.shape[0]
    mask = 0
    for t in terms:
        mask |= TERMS[t]
    score = np.empty(F, np.float64)
    order = np.empty(max(topk, 1), np.int64)
    margin = ctypes.c_double()
    ties = ctypes.c_int()
    k = lib().orc_bucket_scores(_ptr(q), Hq, d, _ptr(counts), _ptr(_c(mean, np.float32)), _ptr(_c(var, np.float32)),
                                F, mask, topk, _ptr(score), _ptr(order), ctypes.byref(margin), ctypes.byref(ties))
    return score, order[:k].copy(), margin.value, ties.value


def qact_scores(q, W, b, query_scale, counts, topk=16):
    """src/prismkv/core.py:131-139 (router="q_activation") -> (score f32[F], order i64, margin)."""
    q = _c(q, np.float32)
    Hq, d = q.shape
    W = _c(W, np.float32)
    F = W.shape[0]
    score = np.empty(F, np.float32)
    order = np.empty(max(F, 1), np.int64)
    margin = ctypes.c_double()
    n = lib().orc_qact_scores(_ptr(q), Hq, d, _ptr(W), _ptr(_c(b, np.float32)), F, float(query_scale),
                              _ptr(_c(counts, np.int64)), topk, _ptr(score), _ptr(order), ctypes.byref(margin))
    return score, order[:n].copy(), margin.value


def norm_top(prod, ln, ct, topk=16):
    """kernels/ppu_8b/route_parallel.cu:13-32 for one group -> (ids i64[16], vals f32[16], raw, margin, ties)."""
    prod = _c(prod, np.float32)
    Hq, F = prod.shape
    ids = np.empty(topk, np.int64)
    vals = np.empty(topk, np.float32)
    raw = ctypes.c_int32()
    margin = ctypes.c_double()
    ties = ctypes.c_int()
    lib().orc_norm_top(_ptr(prod), _ptr(_c(ln, np.float32)), _ptr(_c(ct, np.int32)), Hq, F, topk, _ptr(ids),
                       _ptr(vals), ctypes.byref(raw), ctypes.byref(margin), ctypes.byref(ties))
    return ids, vals, raw.value, margin.value, ties.value


def pack(q_bits):
    """kernels/ppu_8b/pack.cu:3: bf16 Q[rows,d] -> f32 [rows, 2d] = [q, q*q]."""
    q_bits = _c(q_bits, np.uint16)
    rows, d = q_bits.shape
    a = np.empty((rows, 2 * d), np.float32)
    lib().orc_pack(_ptr(q_bits), rows, d, _ptr(a))
    return a


# ---------------------------------------------------------------- stage 2

def select_buckets(order, lists, history, unique_cap=None):
    """src/prismkv/core.py:142-167 -> (ids i64[U], meta dict)."""
    if unique_cap is not None and not 0 <= unique_cap <= 1:
        raise ValueError("unique_cap must be a fraction in [0,1]")
    offsets, ids = lists_to_csr(lists)
    order = _c(order, np.int64)
    out = np.empty(max(history, 1), np.int64)
    feats = np.empty(max(len(order), 1), np.int64)
    nf = ctypes.c_int()
    raw = ctypes.c_int64()
    limit = ctypes.c_int64()
    n = lib().orc_select_buckets(_ptr(order), len(order), _ptr(offsets), _ptr(_c(ids, np.int64)), history,
                                 -1.0 if unique_cap is None else float(unique_cap), _ptr(out), _ptr(feats),
                                 ctypes.byref(nf), ctypes.byref(raw), ctypes.byref(limit))
    return out[:n].copy(), dict(features=feats[:nf.value].tolist(), raw=raw.value, unique=int(n),
                                limit=limit.value, candidate_buckets=len(order))


def build_bits(lists, row_words):
    """kernels/ppu_8b/pack.cu:5 -> uint32 [F, row_words]."""
    offsets, ids = lists_to_csr(lists)
    F = len(lists)
    bits = np.zeros((F, row_words), np.uint32)
    lib().orc_build_bits(_ptr(offsets), _ptr(_c(ids, np.int64)), F, row_words, _ptr(bits))
    return bits


def union_bits(bits, history, features, valid):
    """kernels/ppu_8b/union.cu:14-27 for one group -> int32 ids (ascending)."""
    bits = _c(bits, np.uint32)
    out = np.empty(max(history, 1), np.int32)
    feats = _c(features, np.int64)
    n = lib().orc_union_bits(_ptr(bits), bits.shape[1], history, _ptr(feats), _ptr(_c(valid, np.float32)),
                             len(feats), _ptr(out))
    return out[:n].copy()


# ---------------------------------------------------------------- stage 3

def attend(q, K, V, old_ids, history):
    """src/prismkv/core.py:170-183 in double: softmax over selected rows + tail [H, L)."""
    q = _c(q, np.float32)
    K = _c(K, np.float32)
    V = _c(V, np.float32)
    if K.shape != V.shape or not 0 <= history <= len(K):
        raise ValueError("invalid KV/history")
    Hq, d = q.shape
    ids = _c(old_ids, np.int64)
    out = np.empty((Hq, d), np.float64)
    rc = lib().orc_attend(_ptr(q), Hq, d, _ptr(K), _ptr(V), K.shape[1], len(K), _ptr(ids), len(ids), history,
                          _ptr(out))
    if rc:
        raise ValueError("old_ids must be unique and address old history only")
    return out
