"""Routed-decode benchmark on one MI355X.

Headline workload (the 8B-geometry kernel check, one decode step of a
Qwen3-8B-shaped model): 36 layers x 8 KV groups x 4 query heads, d=128,
F=3000 buckets, Top-16, history H=65536 plus a 256-token generated tail, bf16
K/V ~ N(0,1), fp32 moment tables, bitmaps [8,3000,2048] u32 per layer; every
key joins the buckets of its top-8 ReLU activations of a random SAE
(W_enc ~ N(0,1/128)).  Inputs are generated on the device (synthetic,
seeded) and stay resident in HBM; 36 distinct layers (~17.7 GB) rotate so
nothing is served from the 256 MB Infinity Cache.

A "step" is one decode step through all layers: for every layer the
Native8B call (route: moment scoring + Top-16, union: bitmap OR + compaction,
sparse AV) -- ONE launch per layer, the fused decode kernel -- captured once
in a HIP graph and replayed.  The headline value is the replay time per
layer in microseconds (lower is better); since every layer is one launch of
the decode kernel, it is also that kernel's average launch time, which the
roofline object divides the algorithmic bytes by.

Further stages, each reported as its own key of the same JSON line:
* route / union / attend: the separate entry points in isolated-stage graphs;
* dense: the all-read control at the same history -- every one of the H + T
  rows attended through the same attention kernel (prismkv_attend with ids
  0..H-1), 36 layers in a graph -- and the sparse / dense time ratio;
* long_history (configuration 4): H=131072 with the tail at 4096, 12
  distinct layers chained to 36 launches, plus the amortised index update of
  a 1024-token block on a 131072-token table;
* capped (configuration 5): H=262144 keys from a 64-component Gaussian
  mixture (sigma 0.3) indexed on the device, strict unique cap H/16, the
  capped step (route, budgeted walk, union + attention: three launches per
  layer) for 12 distinct layers chained to 36, one HIP graph, with the
  per-stage launch times and HBM rates, and the uncapped single launch at the
  same history beside it;
* update / build: the index update (N=1024, 4096) and the prefill build at 64K.

The CPU baseline is the torch-CPU restatement of the reference's per-group
decode step (oracle/torch_cpu.py: route, union walk, attention, 8 groups) on
layer 0 of the headline workload, with torch.set_num_threads(all host cores)
and with one thread, median of 7 after 2 warm-ups; the configuration-1
replay shape and the reference's append_index per 1024-token block are timed
the same way, and the C oracle beside them.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0
METRIC = "routed decode µs/layer at 64K history (8 groups); per-stage HBM GB/s vs peak"
PPU_US_PER_LAYER_64K = 108.3  # whole sparse chain, PPU-ZW810 (tail 8)
G, HQ, D, F, TOPK = 8, 4, 128, 3000, 16
# HBM bytes per launch from the two counter passes (FETCH_SIZE, WRITE_SIZE)
# over this workload, each scaled by what the counter reads for a 1 GiB
# streaming kernel; measured at H=65536, T=256 only.
TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "decode_kernel_64k_hbm_traffic.md")
STAGE_KERNEL = {"decode": "decode_kernel"}


def nbytes(t):
    """Bytes of a workspace tensor (the work_bytes argument beside its pointer)."""
    return t.numel() * t.element_size()
DEFAULT_STAGES = "chain,route,union,attend,dense,update,build,copy,long_history,capped,tails,amortised"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=36)
    p.add_argument("--history", type=int, default=65536)
    p.add_argument("--tail", type=int, default=256)
    p.add_argument("--seed", type=int, default=2)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--update-blocks", default="1024,4096",
                   help="block sizes of the amortised index-update timing (tokens per append)")
    p.add_argument("--stages", default=DEFAULT_STAGES, help="comma list of timed regions (for profiling runs)")
    p.add_argument("--library", default=None,
                   help="a libprismkv_hip.so other than the in-tree one (A/B builds of prismkv_amd.build)")
    return p.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def stream():
    return torch.cuda.current_stream().cuda_stream


@torch.no_grad()
def make_layer(lib_path, layer, H, T, seed, device, capacity=None):
    """One layer: K/V/Q and its 8 group indices built on the device."""
    from prismkv_amd import Native8B
    gen = torch.Generator(device=device)
    gen.manual_seed(seed * 1000 + layer)
    k = torch.randn(G, H + T, D, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn(G, H + T, D, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
    q = torch.randn(G, HQ, D, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
    counts = torch.zeros(G, F, dtype=torch.int64, device=device)
    mean = torch.zeros(G, F, D, device=device)
    var = torch.zeros(G, F, D, device=device)
    csr, offs = [], []
    for g in range(G):
        W = torch.randn(F, D, generator=gen, device=device) / D ** 0.5
        keys = k[g, :H].float()
        toks, feats = [], []
        for lo in range(0, H, 16384):
            a = keys[lo:lo + 16384] @ W.T
            val, idx = a.topk(8, dim=1)
            keep = val > 0
            rows = torch.arange(lo, lo + len(a), device=device)[:, None].expand_as(idx)
            toks.append(rows[keep])
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
    op = Native8B.from_tables(H, counts, mean, var, csr, torch.stack(offs), lib_path, capacity=capacity)
    return op, q, k, v


@torch.no_grad()
def make_mixture_layer(lib_path, layer, H, T, seed, device, unique_cap):
    """One layer of the stress configuration: keys from a 64-component
    Gaussian mixture (centers ~ N(0, I), uniform weights, sigma 0.3), V and Q
    ~ N(0, 1), indexed on the device (build_index with a random SAE per
    group, global budget 8 H); strict unique cap."""
    from prismkv_amd import Native8B
    gen = torch.Generator(device=device)
    gen.manual_seed(seed * 7717 + layer)
    centers = torch.randn(G, 64, D, generator=gen, device=device)
    comp = torch.randint(0, 64, (G, H + T), generator=gen, device=device)
    k = torch.randn(G, H + T, D, generator=gen, device=device).mul_(0.3)
    k.add_(torch.gather(centers, 1, comp[..., None].expand(-1, -1, D)))
    k = k.to(torch.bfloat16)
    v = torch.randn(G, H + T, D, generator=gen, device=device).to(torch.bfloat16)
    q = torch.randn(G, HQ, D, generator=gen, device=device).to(torch.bfloat16)
    W = torch.randn(G, F, D, generator=gen, device=device) / D ** 0.5
    b = torch.zeros(G, F, device=device)
    op = Native8B.from_keys(k, H, W, b, torch.ones(G), 8, lib_path, capacity=H + T, unique_cap=unique_cap)
    del centers, comp, W, b
    return op, q, k, v


def measured_traffic(stage, H, T):
    """Counter-derived HBM bytes per launch of the stage's kernel, or None."""
    if (H, T) != (65536, 256) or stage not in STAGE_KERNEL or not os.path.exists(TRAFFIC_PROFILE):
        return None
    with open(TRAFFIC_PROFILE) as fh:
        for line in fh:
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == STAGE_KERNEL[stage]:
                return int(parts[2])
    return None


def graph_time(fn, steps, warmup):
    """Capture fn once, replay; returns (ms per replay by events, ms per replay wall, graph)."""
    cur = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    with torch.cuda.stream(side):
        fn()
    cur.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return e0.elapsed_time(e1) / steps, wall, graph


def rate(nbytes, us):
    gbs = nbytes / (us * 1e-6) / 1e9
    return dict(us_per_launch=round(us, 3), algorithmic_bytes=int(nbytes), achieved_GBps=round(gbs, 1),
                frac_of_peak=round(gbs / HBM_PEAK_GBS, 4))


def route_bytes():
    return G * F * (2 * D * 4 + 4) + G * HQ * D * 2 + G * TOPK * 12 + G * 4


def stage_bytes(ops, H, T):
    """Algorithmic HBM bytes per launch (8 groups of one layer), averaged over layers."""
    nw = (H + 31) // 32
    unions, avs, uniq = [], [], []
    for op in ops:
        u = op.count.cpu().numpy().astype(np.int64)
        nsel = (op.valid.cpu().numpy() > 0).sum(1)
        unions.append(int((nsel * nw * 4 + u * 4 + 4).sum() + G * TOPK * 12))
        avs.append(int(((u + T) * 2 * D * 2 + u * 4 + 4).sum() + 2 * G * HQ * D * 2))
        uniq.append(u.mean())
    return route_bytes(), float(np.mean(unions)), float(np.mean(avs)), float(np.mean(uniq))


def chain_of(layers, n):
    """n decode launches cycling over the given layers."""
    def run():
        for i in range(n):
            op, q, k, v = layers[i % len(layers)]
            op(q, k, v)
    return run


@torch.no_grad()
def dense_control(layers, H, T, steps, warmup):
    """All-read control: the attention kernel over every history row plus the
    tail (ids 0..H-1) for each layer, in one graph; returns µs per layer."""
    op0 = layers[0][0]
    lib = op0.lib
    device = op0.out.device
    ids = torch.arange(H, dtype=torch.int32, device=device).repeat(G, 1).contiguous()
    count = torch.full((G,), H, dtype=torch.int32, device=device)
    splits = 256 // G  # one workgroup per CU over the 8 groups
    work = torch.zeros(lib.query("prismkv_attend_work_bytes", G, splits), dtype=torch.uint8, device=device)
    out = torch.zeros(G, HQ, D, dtype=torch.bfloat16, device=device)

    def run():
        for _, q, k, v in layers:
            lib.call("prismkv_attend", q.data_ptr(), k.data_ptr(), v.data_ptr(), ids.data_ptr(), count.data_ptr(),
                     work.data_ptr(), out.data_ptr(), G, H, T, k.stride(0), v.stride(0), H, splits, nbytes(work),
                     stream=stream())
    ms, _, _ = graph_time(run, steps, warmup)
    us = ms * 1e3 / len(layers)
    dense_bytes = G * (H + T) * 2 * D * 2 + G * H * 4 + 2 * G * HQ * D * 2
    return us, dense_bytes


@torch.no_grad()
def update_timing(lib_path, H, blocks, steps, warmup, seed, device):
    """Amortised index update: one prismkv_update launch sequence per replay
    (encode, BatchTopK threshold, bitmap append, moment merge for 8 groups),
    indexing a block of N keys at history H - N of a dedicated table (so the
    decode tables are untouched).  Every replay indexes the same block."""
    from prismkv_amd import Native8B
    gen = torch.Generator(device=device)
    gen.manual_seed(seed * 7919)
    out = {}
    k = torch.randn(G, H, D, generator=gen, device=device).to(torch.bfloat16)
    W = torch.randn(G, F, D, generator=gen, device=device) / D ** 0.5
    b = torch.zeros(G, F, device=device)
    for N in blocks:
        h0 = H - N
        counts = torch.full((G, F), 8, dtype=torch.int64, device=device)
        mean = torch.randn(G, F, D, generator=gen, device=device) * 0.1
        var = torch.rand(G, F, D, generator=gen, device=device)
        csr = torch.zeros(G, 1, dtype=torch.int32, device=device)
        offs = torch.zeros(G, F + 1, dtype=torch.int32, device=device)
        op = Native8B.from_tables(h0, counts, mean, var, csr, offs, lib_path, capacity=H,
                                  center=k[:, :h0].float().mean(1))
        op.set_encoder_tables(W, b, torch.ones(G), 8)
        op.append(k, N)  # allocates the workspace; history -> H
        torch.cuda.synchronize()

        def once():
            op.lib.call("prismkv_update", k.data_ptr(), op.W_enc.data_ptr(), op.b_enc.data_ptr(),
                        op.center.data_ptr(), op.key_scale.data_ptr(), op.bits.data_ptr(), op.n.data_ptr(),
                        op.moments.data_ptr(), op.update_work.data_ptr(), G, h0, N, 8, k.stride(0), op.row_words,
                        nbytes(op.update_work), stream=stream())
        ms, _, _ = graph_time(once, steps, warmup)
        us = ms * 1e3
        flops = 2.0 * G * N * F * D
        out[str(N)] = dict(us_per_block=round(us, 2), us_per_token_per_layer=round(us / N, 4),
                           encode_gflop=round(flops / 1e9, 2), encode_tflops_if_alone=round(flops / (us * 1e-6) / 1e12, 2))
        log(f"update H={H} N={N}: {us:.1f} us per block ({us / N:.3f} us per token per layer, amortised)")
        del op
    del k, W, b
    torch.cuda.empty_cache()
    return out


@torch.no_grad()
def build_timing(lib_path, H, steps, warmup, seed, device):
    """Prefill index build of one layer: one prismkv_build per replay (center,
    bitmap clear, encode, exact BatchTopK with budget 8 H, bitmap set,
    per-bucket two-pass moments) for the 8 groups' K rows [0, H), into the
    tables of a dedicated instance."""
    from prismkv_amd import Native8B
    gen = torch.Generator(device=device)
    gen.manual_seed(seed * 104729)
    k = torch.randn(G, H, D, generator=gen, device=device).to(torch.bfloat16)
    W = torch.randn(G, F, D, generator=gen, device=device) / D ** 0.5
    b = torch.zeros(G, F, device=device)
    op = Native8B.from_keys(k, H, W, b, torch.ones(G), 8, lib_path, keep_activations=True)
    torch.cuda.synchronize()

    def once():
        op.lib.call("prismkv_build", k.data_ptr(), op.W_enc.data_ptr(), op.b_enc.data_ptr(), op.center.data_ptr(),
                    op.key_scale.data_ptr(), op.bits.data_ptr(), op.n.data_ptr(), op.moments.data_ptr(),
                    op.build_work.data_ptr(), G, op.build_batch, H, 8, 1, k.stride(0), op.row_words,
                    nbytes(op.build_work), stream=stream())
    ms, _, _ = graph_time(once, max(2, steps // 4), max(1, warmup // 4))
    flops = 2.0 * G * H * F * D
    out = dict(history=H, ms_per_layer=round(ms, 3), groups_per_batch=op.build_batch,
               memberships_per_group=int(op.n[0].sum()), encode_gflop=round(flops / 1e9, 1),
               encode_tflops_if_alone=round(flops / (ms * 1e-3) / 1e12, 2))
    log(f"build H={H}: {ms:.2f} ms per layer (8 groups)")
    del op, k, W, b
    torch.cuda.empty_cache()
    return out


@torch.no_grad()
def long_history(lib_path, steps, warmup, seed, device, layers_total, replicas=12, H=131072, T=4096):
    """Configuration 4: decode at H=131072 with a 4096-token tail (12
    distinct layers chained to `layers_total` launches), and the amortised
    update of one 1024-token block on a 131072-token table."""
    log(f"long history: building {replicas} layers H={H} T={T} ...")
    layers = [make_layer(lib_path, 100 + i, H, T, seed, device) for i in range(replicas)]
    torch.cuda.synchronize()
    run = chain_of(layers, layers_total)
    run()
    torch.cuda.synchronize()
    errors = max(l[0].decode_errors() for l in layers)
    ms, _, _ = graph_time(run, steps, warmup)
    us = ms * 1e3 / layers_total
    r, u, a, uniq = stage_bytes([l[0] for l in layers], H, T)
    out = dict(history=H, tail=T, layers=layers_total, distinct_layers=replicas,
               decode=rate(r + u + a, us), mean_unique_ids_per_group=round(uniq, 1), wait_errors=errors)
    log(f"long history: {us:.2f} us/layer decode at H={H} T={T}")
    del layers, run
    torch.cuda.empty_cache()
    upd = update_timing(lib_path, H, [1024], steps, warmup, seed, device)["1024"]
    out["update_1024"] = upd
    # per token and layer: one decode plus 1/1024 of a block update
    out["us_per_token_per_layer_with_update"] = round(us + upd["us_per_block"] / 1024, 3)
    return out


@torch.no_grad()
def tails(lib_path, steps, warmup, seed, device, layers_total, H=65536, tails_=(2048, 4096)):
    """The headline history with the longer tails the update policy leaves:
    with the reference's default interval of 4096 tokens
    (configs/submitted_8b.json:14) the unindexed tail runs from 0 to 4096
    rows between updates.  36 distinct layers built with the longest tail;
    each tail length is timed on views of the same layers."""
    T_max = max(tails_)
    log(f"tails: building {layers_total} layers H={H} T={T_max} ...")
    layers = [make_layer(lib_path, 200 + i, H, T_max, seed, device) for i in range(layers_total)]
    torch.cuda.synchronize()
    out = {}
    for T in tails_:
        views = [(op, q, k[:, :H + T], v[:, :H + T]) for op, q, k, v in layers]
        run = chain_of(views, layers_total)
        run()
        torch.cuda.synchronize()
        errors = max(l[0].decode_errors() for l in views)
        ms, _, _ = graph_time(run, steps, warmup)
        us = ms * 1e3 / layers_total
        r, u, a, uniq = stage_bytes([l[0] for l in views], H, T)
        out[str(T)] = dict(decode=rate(r + u + a, us), mean_unique_ids_per_group=round(uniq, 1), wait_errors=errors)
        log(f"tails: {us:.2f} us/layer decode at H={H} T={T}")
    del layers
    torch.cuda.empty_cache()
    return dict(history=H, layers=layers_total, by_tail=out)


@torch.no_grad()
def amortised(lib_path, steps, warmup, seed, device, layers_total, replicas=12, histories=(32768, 65536),
              intervals=(512, 2048, 4096)):
    """Decode with the index update amortised, as the reference reports it
    (reviewer_guide/results/hyperparameter_sensitivity/README.md:49-58, the
    update intervals 512 / 2048 / 4096 at 32K and 64K): per token and layer,
    one decode at the window's mean tail (interval / 2 rows; the decode time
    grows linearly with the tail) plus 1/interval of one block update of
    `interval` keys on a table of that history."""
    out = {}
    for H in histories:
        T_max = max(intervals) // 2
        log(f"amortised: building {replicas} layers H={H} T={T_max} ...")
        layers = [make_layer(lib_path, 300 + i, H, T_max, seed, device) for i in range(replicas)]
        torch.cuda.synchronize()
        dec = {}
        for n in intervals:
            T = n // 2
            views = [(op, q, k[:, :H + T], v[:, :H + T]) for op, q, k, v in layers]
            run = chain_of(views, layers_total)
            run()
            torch.cuda.synchronize()
            ms, _, _ = graph_time(run, steps, warmup)
            dec[n] = ms * 1e3 / layers_total
        del layers, views, run
        torch.cuda.empty_cache()
        upd = update_timing(lib_path, H, list(intervals), steps, warmup, seed, device)
        for n in intervals:
            u = upd[str(n)]["us_per_block"]
            out[f"{H}/{n}"] = dict(history=H, interval=n, decode_us_per_layer_at_mean_tail=round(dec[n], 3),
                                   mean_tail=n // 2, update_us_per_block=u,
                                   update_us_per_token_per_layer=round(u / n, 4),
                                   us_per_token_per_layer=round(dec[n] + u / n, 3))
            log(f"amortised H={H} interval {n}: decode {dec[n]:.2f} + update {u / n:.3f} us per token and layer")
    return out


@torch.no_grad()
def capped(lib_path, steps, warmup, seed, device, layers_total, replicas=12, H=262144, T=256, cap=1 / 16):
    """Configuration 5: the capped step at H=262144 over mixture keys, one
    launch per layer (prismkv_decode_capped: route, the budgeted walk spread
    over the group's workgroups, union + attention), 12 distinct layers
    chained to `layers_total`, in one graph; for comparison the same step as
    three launches (prismkv_route_single, prismkv_select_cap_n,
    prismkv_union_attend) and per-stage graphs of each; the uncapped single
    launch at the same history."""
    log(f"capped: building {replicas} mixture-key layers H={H} T={T} on the device ...")
    t0 = time.perf_counter()
    layers = [make_mixture_layer(lib_path, 200 + i, H, T, seed, device, cap) for i in range(replicas)]
    torch.cuda.synchronize()
    log(f"capped: built in {time.perf_counter() - t0:.1f}s")
    nw = (H + 31) // 32
    limit = int(H * cap)
    # byte model from one eager pass: ranked and kept rows per group
    ranked, kept, uniq = [], [], []
    for op, q, k, v in layers:
        op.unique_cap = None
        op.lib.call("prismkv_route_single", q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(),
                    op.decode_work.data_ptr(), op.features.data_ptr(), op.valid.data_ptr(), op.raw.data_ptr(), G,
                    nbytes(op.decode_work), stream=stream())
        ranked.append((op.valid > 0).sum(1).cpu().numpy())
        op.unique_cap = cap
        op(q, k, v)
        kept.append((op.valid > 0).sum(1).cpu().numpy())
        uniq.append(op.count.cpu().numpy().astype(np.int64))
    torch.cuda.synchronize()
    errors = max(l[0].decode_errors() for l in layers)
    b_route = route_bytes()
    b_cap = float(np.mean([(r * nw * 4).sum() + G * TOPK * 12 for r in ranked]))
    b_ua = float(np.mean([(kp * nw * 4 + u * 4 + 4 + (u + T) * 2 * D * 2).sum() + 2 * G * HQ * D * 2
                          for kp, u in zip(kept, uniq)]))
    # the one launch reads each ranked row once (the walk's words are the union's)
    b_one = b_route + float(np.mean([(r * nw * 4).sum() for r in ranked])) + float(np.mean(
        [(u * 4 + 4 + (u + T) * 2 * D * 2).sum() + 2 * G * HQ * D * 2 for u in uniq]))

    def step():
        for i in range(layers_total):
            op, q, k, v = layers[i % replicas]
            op(q, k, v)
    ms, _, _ = graph_time(step, steps, warmup)
    us = ms * 1e3 / layers_total

    def stage(fn):
        def run():
            for i in range(layers_total):
                fn(*layers[i % replicas])
        sm, _, _ = graph_time(run, steps, warmup)
        return sm * 1e3 / layers_total

    def route_only(op, q, k, v):
        op.lib.call("prismkv_route_single", q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(),
                    op.decode_work.data_ptr(), op.features.data_ptr(), op.valid.data_ptr(), op.raw.data_ptr(), G,
                    nbytes(op.decode_work), stream=stream())

    def walk_only(op, q, k, v):
        op.lib.call("prismkv_select_cap_n", op.bits.data_ptr(), op.n.data_ptr(), op.features.data_ptr(),
                    op.valid.data_ptr(), op.raw.data_ptr(), G, op.history, limit, op.row_words, TOPK,
                    stream=stream())

    def union_attend_only(op, q, k, v):
        op.lib.call("prismkv_union_attend", q.data_ptr(), op.bits.data_ptr(), k.data_ptr(), v.data_ptr(),
                    op.decode_work.data_ptr(), op.features.data_ptr(), op.valid.data_ptr(), op.ids.data_ptr(),
                    op.count.data_ptr(), op.out.data_ptr(), G, op.history, k.shape[1] - op.history, op.capacity,
                    op.row_words, k.stride(0), v.stride(0), op.capacity, nbytes(op.decode_work), stream=stream())
    us_route = stage(route_only)
    # the walk re-reads the route's ranking: restore it before timing the walk
    for op, q, k, v in layers:
        route_only(op, q, k, v)
    us_walk = stage(lambda op, q, k, v: (route_only(op, q, k, v), walk_only(op, q, k, v))) - us_route
    for op, q, k, v in layers:
        op(q, k, v)  # the capped selection in features / valid again
    us_ua = stage(union_attend_only)
    us_three = stage(lambda op, q, k, v: (route_only(op, q, k, v), walk_only(op, q, k, v),
                                          union_attend_only(op, q, k, v)))
    # the uncapped single launch at the same history
    for op, _, _, _ in layers:
        op.unique_cap = None
    run = chain_of(layers, layers_total)
    run()
    torch.cuda.synchronize()
    um, _, _ = graph_time(run, steps, warmup)
    us_uncapped = um * 1e3 / layers_total
    r, u, a, uniq_u = stage_bytes([l[0] for l in layers], H, T)
    out = dict(history=H, tail=T, unique_cap=cap, limit=limit, layers=layers_total, distinct_layers=replicas,
               keys="64-component Gaussian mixture, sigma 0.3, device-built index (global budget 8H)",
               us_per_layer=round(us, 3), ms_per_step=round(ms, 4), launches_per_layer=1,
               decode_capped=rate(b_one, us), mean_ranked_buckets=round(float(np.mean(ranked)), 2),
               mean_kept_buckets=round(float(np.mean(kept)), 2),
               mean_unique_ids_per_group=round(float(np.mean(uniq)), 1), wait_errors=errors,
               three_launches=dict(us_per_layer=round(us_three, 3),
                                   stages={"route_kernel": rate(b_route, us_route), "cap_walk": rate(b_cap, us_walk),
                                           "union_attend": rate(b_ua, us_ua)}),
               uncapped_single_launch=dict(rate(r + u + a, us_uncapped),
                                           mean_unique_ids_per_group=round(uniq_u, 1)))
    log(f"capped: {us:.2f} us/layer in one launch; three launches {us_three:.2f} (route {us_route:.2f} + walk "
        f"{us_walk:.2f} + union/attend {us_ua:.2f}); uncapped single launch {us_uncapped:.2f}")
    del layers, run
    torch.cuda.empty_cache()
    return out


def host_cpu():
    """(model name, logical CPUs of the host, threads this process may use)."""
    model, cpus = None, os.cpu_count()
    try:
        text = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in text.splitlines():
            key, _, val = line.partition(":")
            if key.strip() == "Model name":
                model = val.strip()
            elif key.strip() == "CPU(s)":
                cpus = int(val.strip())
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    usable = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        usable = min(usable, int(os.environ["OMP_NUM_THREADS"]))
    return model, cpus, max(1, usable)


def median_time(fn, warmup=2, reps=7):
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)) * 1e6


@torch.no_grad()
def cpu_baseline(op, q, k, v, H, threads):
    """The torch-CPU restatement of the reference's decode step (route, union
    walk, attention) for the 8 groups of layer 0 (configuration 2), the
    configuration-1 replay shape, and append_index of one 1024-token block
    (one group, x8), each with torch.set_num_threads(threads) and 1 thread;
    plus the C oracle's route + union + attention on layer 0 (1 thread)."""
    import oracle
    from oracle import cases, torch_cpu as tc
    oracle.build()
    idx = op.export_indices()
    kc, vc, qc = k.cpu(), v.cpu(), q.cpu()
    groups = [(qc[g], idx[g].counts.cpu(), idx[g].mean.cpu(), idx[g].variance.cpu(),
               [l.long() for l in idx[g].lists], kc[g], vc[g]) for g in range(G)]
    rep = cases.replay_case(seed=5, H=1024, T=32, bf16=False)
    rgroups = [(torch.from_numpy(rep["q"][g]), torch.from_numpy(i.counts), torch.from_numpy(i.mean),
                torch.from_numpy(i.variance), [torch.from_numpy(np.asarray(l, np.int64)) for l in i.lists],
                torch.from_numpy(rep["k"][g]), torch.from_numpy(rep["v"][g])) for g, i in enumerate(rep["indices"])]
    upd = cases.update_case("random", H=256, N=1024, T=0, seed=23)  # a 1024-key block on a 256-token index
    ui = upd["indices"][0]
    ukeys = torch.from_numpy(oracle.bf16_to_f32(upd["k"][0, 256:1280]))
    ulists = [torch.from_numpy(np.asarray(l, np.int64)) for l in ui.lists]

    def layer(gs, hist):
        for qg, cg, mg, vg, lg, kg, vv in gs:
            tc.decode_group(qg, cg, mg, vg, lg, kg, vv, hist)

    def append():
        tc.append_block(torch.from_numpy(ui.counts), torch.from_numpy(ui.mean), torch.from_numpy(ui.variance),
                        ulists, 256, torch.from_numpy(ui.center), ukeys, torch.from_numpy(upd["W"][0]),
                        torch.from_numpy(upd["b"][0]), float(upd["scale"][0]), 8)

    old = torch.get_num_threads()
    res = {}
    try:
        for n in (threads, 1):
            torch.set_num_threads(n)
            res[n] = dict(layer=median_time(lambda: layer(groups, H)), replay=median_time(lambda: layer(rgroups, 1024)),
                          append=median_time(append) * G)
            log(f"cpu baseline ({n} threads): {res[n]['layer']:.0f} us/layer at H={H}, "
                f"{res[n]['replay']:.0f} us/layer replay shape, {res[n]['append']:.0f} us per 1024-block update")
    finally:
        torch.set_num_threads(old)
    # the C oracle (fp64 accumulation), route + union + attention of layer 0, one thread
    counts = op.n[:, :F].cpu().numpy().astype(np.int64)
    from prismkv_amd import untile_moments
    mean, var = (x.cpu().numpy() for x in untile_moments(op.moments))
    bits = op.bits.cpu().numpy().view(np.uint32)
    qf, kf, vf = qc.float().numpy(), kc.float().numpy(), vc.float().numpy()

    def c_layer():
        for g in range(G):
            _, order, _, _ = oracle.bucket_scores(qf[g], counts[g], mean[g], var[g])
            feats = np.zeros(TOPK, np.int64)
            feats[:len(order)] = order
            ids = oracle.union_bits(bits[g], H, feats, (np.arange(TOPK) < len(order)).astype(np.float32))
            oracle.attend(qf[g], kf[g], vf[g], ids, H)
    c_us = median_time(c_layer, warmup=1, reps=3)
    log(f"cpu baseline: C oracle {c_us:.0f} us/layer (1 thread)")
    return res, c_us


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one MI355X only; --gpus {a.gpus} is not supported (this path shards by KV "
              f"group or layer with no exchange; see the design notes).", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    from prismkv_amd import _lib
    lib_path = a.library or _lib.DEFAULT_LIBRARY
    _lib.load(lib_path)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    stages = set(a.stages.split(","))
    H, T = a.history, a.tail
    if not stages & {"chain", "route", "union", "attend", "dense"}:
        # a profiling run of the other configurations alone: no headline workload
        a.no_cpu_baseline = True
        out = dict(long_history=long_history(lib_path, a.steps, a.warmup, a.seed, device, a.layers)
                   if "long_history" in stages else None,
                   capped=capped(lib_path, a.steps, a.warmup, a.seed, device, a.layers) if "capped" in stages else None,
                   update=update_timing(lib_path, H, [int(x) for x in a.update_blocks.split(",") if x], a.steps,
                                        a.warmup, a.seed, device) if "update" in stages else None,
                   build=build_timing(lib_path, H, a.steps, a.warmup, a.seed, device) if "build" in stages else None,
                   tails=tails(lib_path, a.steps, a.warmup, a.seed, device, a.layers, H) if "tails" in stages else None,
                   amortised=amortised(lib_path, a.steps, a.warmup, a.seed, device, a.layers)
                   if "amortised" in stages else None)
        print(json.dumps(out), flush=True)
        return
    log(f"building {a.layers} layers H={H} T={T} ...")
    t0 = time.perf_counter()
    layers = [make_layer(lib_path, i, H, T, a.seed, device) for i in range(a.layers)]
    torch.cuda.synchronize()
    log(f"built in {time.perf_counter() - t0:.1f}s; mem {torch.cuda.memory_allocated() / 2**30:.1f} GiB")

    def chain():  # the decode step: Native8B.__call__ = route + attention (fused path, 1 launch per layer)
        for op, q, k, v in layers:
            op(q, k, v)

    def route_only():  # Native8B.route(): moment scoring, Top-16, union and ids in one launch
        for op, q, k, v in layers:
            op.route(q)

    def union_only():
        for op, q, k, v in layers:
            op.lib.call("prismkv_union", op.bits.data_ptr(), op.features.data_ptr(), op.valid.data_ptr(),
                        op.union_work.data_ptr(), op.ids.data_ptr(), op.count.data_ptr(), G, op.history,
                        op.row_words, op.capacity, nbytes(op.union_work), stream=stream())

    def attend_only():
        for op, q, k, v in layers:
            op.attention(q, k, v)

    chain()  # populate ids/count for the byte model and the stage graphs
    torch.cuda.synchronize()
    ms, wall, _ = graph_time(chain, a.steps, a.warmup) if "chain" in stages else (float("nan"),) * 3
    log(f"chain: {ms:.4f} ms/step events, {wall:.4f} ms/step wall")
    per_stage = {}
    if "chain" in stages:
        per_stage["decode"] = ms * 1e3 / a.layers  # one decode_kernel launch per layer
    for name, fn in (("route", route_only), ("union", union_only), ("attend", attend_only)):
        if name in stages:
            sm, _, _ = graph_time(fn, a.steps, a.warmup)
            per_stage[name] = sm * 1e3 / a.layers
            log(f"{name}: {per_stage[name]:.2f} us/launch")
    chain()
    torch.cuda.synchronize()
    wait_errors = max(l[0].decode_errors() for l in layers)
    b_route, b_union, b_av, uniq = stage_bytes([l[0] for l in layers], H, T)
    stage_nbytes = {"decode": b_route + b_union + b_av, "route": b_route + b_union, "union": b_union,
                    "attend": b_av}
    stage_report = {name: rate(stage_nbytes[name], us) for name, us in per_stage.items()}
    dense = None
    if "dense" in stages:
        d_us, d_bytes = dense_control(layers, H, T, a.steps, a.warmup)
        dense = dict(rate(d_bytes, d_us), rows_per_group=H + T,
                     kernel="prismkv_attend over ids 0..H-1 plus the tail (the all-read control)")
        if "decode" in per_stage:
            dense["sparse_over_dense_time"] = round(per_stage["decode"] / d_us, 4)
            dense["dense_over_sparse_time"] = round(d_us / per_stage["decode"], 3)
        log(f"dense control: {d_us:.2f} us/layer")
    copy_gbs = None
    if "copy" in stages:
        # a plain streaming kernel of known size (1 GiB read + 1 GiB written): the
        # attainable-bandwidth probe, and the reference for HBM byte counters
        src = torch.ones(2 ** 28, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            torch.neg(src, out=dst)
        e1.record()
        torch.cuda.synchronize()
        copy_gbs = 2 * 2 ** 30 * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9
        log(f"copy probe: {copy_gbs:.0f} GB/s (read+write)")
        del src, dst
    cpu = None
    if not a.no_cpu_baseline:
        model, cpus, threads = host_cpu()
        op, q, k, v = layers[0]
        res, c_us = cpu_baseline(op, q, k, v, H, threads)
        cpu = dict(value=round(res[threads]["layer"], 1), unit="us/layer", cores=threads, kind="port",
                   sample=f"layer 0 of the workload (8 groups, H={H}, T={T}): the torch-CPU restatement of the "
                          f"reference decode step (route, union walk, attention per group), "
                          f"torch.set_num_threads({threads}), median of 7 after 2 warm-ups",
                   cpu_model=model, host_logical_cpus=cpus, value_1_thread=round(res[1]["layer"], 1),
                   replay_shape_us_per_layer={str(n): round(r["replay"], 1) for n, r in res.items()},
                   append_1024_block_us={str(n): round(r["append"], 1) for n, r in res.items()},
                   c_oracle_us_per_layer_1_thread=round(c_us, 1))
        del op, q, k, v
    update = None
    if "update" in stages:
        blocks = [int(x) for x in a.update_blocks.split(",") if x]
        update = update_timing(lib_path, H, blocks, a.steps, a.warmup, a.seed, device)
    build = build_timing(lib_path, H, a.steps, a.warmup, a.seed, device) if "build" in stages else None
    fused = [n for n in ("decode",) if n in stage_report]
    dominant = max(fused or stage_report, key=lambda n: stage_report[n]["us_per_launch"]) if stage_report else None
    roofline = None
    if dominant:
        d = stage_report[dominant]
        traffic = measured_traffic(dominant, H, T)
        roofline = dict(bound="hbm", achieved=d["achieved_GBps"], peak=HBM_PEAK_GBS, unit="GB/s",
                        frac=d["frac_of_peak"], traffic=traffic,
                        traffic_source=None if traffic is None else
                        "profile-derived, not collected by this run: FETCH_SIZE and WRITE_SIZE passes over this "
                        "workload, scaled by the copy kernel's factors, which the dense control's gather of known "
                        "size confirms to 1.1% (profiles/decode_kernel_64k_hbm_traffic.md)",
                        kernel=STAGE_KERNEL.get(dominant, dominant), algorithmic_bytes=d["algorithmic_bytes"])
    n_layers = a.layers
    del layers
    torch.cuda.empty_cache()
    long_h = long_history(lib_path, a.steps, a.warmup, a.seed, device, n_layers) if "long_history" in stages else None
    cap = capped(lib_path, a.steps, a.warmup, a.seed, device, n_layers) if "capped" in stages else None
    tail_lines = tails(lib_path, a.steps, a.warmup, a.seed, device, n_layers, H) if "tails" in stages else None
    amort = amortised(lib_path, a.steps, a.warmup, a.seed, device, n_layers) if "amortised" in stages else None
    value = ms * 1e3 / a.layers
    result = {
        "metric": METRIC, "value": round(value, 3), "unit": "us/layer", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": round(value / PPU_US_PER_LAYER_64K, 4), "dtype": "bf16",
        "dtype_detail": "moment scoring and selection in fp32; QK on bf16 MFMA with fp32 accumulation; "
                        "P split into a bf16 head and a bf16 remainder (about 16 significant bits) for the PV "
                        "MFMA, fp32 accumulation; bf16 output",
        "data": "synthetic",
        "config": {"workload": f"8B-geometry routed decode, {a.layers} layers x 8 KV groups x 4 Q heads, d=128, "
                               f"F=3000, Top-16, H={H} + {T} tail, bf16 KV, per-key top-8 SAE membership",
                   "layers": a.layers, "groups": G, "history": H, "tail": T,
                   "kv_dtype": "bf16", "mean_unique_ids_per_group": round(uniq, 1), "parallelism": "single GPU"},
        "wall_ms_per_step": round(wall, 4), "wait_errors": wait_errors, "stages": stage_report, "dense": dense,
        "copy_probe_GBps": copy_gbs and round(copy_gbs, 1), "update": update, "build": build,
        "long_history": long_h, "capped": cap, "tails": tail_lines, "amortised": amort, "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
