"""Routed-decode benchmark on one MI355X.

Workload (the 8B-geometry kernel check, one decode step of a Qwen3-8B-shaped
model): 36 layers x 8 KV groups x 4 query heads, d=128, F=3000 buckets,
Top-16, history H=65536 plus a 256-token generated tail, bf16 K/V ~ N(0,1),
fp32 moment tables, bitmaps [8,3000,2048] u32 per layer; every key joins the
buckets of its top-8 ReLU activations of a random SAE (W_enc ~ N(0,1/128)).
Inputs are generated on the device (synthetic, seeded) and stay resident in
HBM; 36 distinct layers (~17.7 GB) rotate so nothing is served from the
256 MB Infinity Cache.

A "step" is one decode step through all layers: for every layer the
Native8B call (route: moment scoring + Top-16, union: bitmap OR + compaction,
sparse AV) -- ONE launch per layer, the fused decode kernel -- captured once
in a HIP graph and replayed.  The headline value is the replay time per
layer in microseconds (lower is better); since every layer is one launch of
the decode kernel, it is also that kernel's average launch time, which the
roofline object divides the algorithmic bytes by.  The separate
route (one launch) / union / attend entry points are timed in isolated-stage
graphs too.  The CPU baseline times the C oracle on a bounded sample of the
same layer workload: one KV group per host thread (8 threads), and on one
thread beside it.
"""
from __future__ import annotations

import argparse
import json
import os
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


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=36)
    p.add_argument("--history", type=int, default=65536)
    p.add_argument("--tail", type=int, default=256)
    p.add_argument("--seed", type=int, default=2)
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU-baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--update-blocks", default="1024,4096",
                   help="block sizes of the amortised index-update timing (tokens per append)")
    p.add_argument("--stages", default="chain,route,union,attend,update,build,copy",
                   help="comma list of timed regions (for profiling runs)")
    return p.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


@torch.no_grad()
def make_layer(lib_path, layer, H, T, seed, device):
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
    op = Native8B.from_tables(H, counts, mean, var, csr, torch.stack(offs), lib_path)
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
    """Capture fn once, replay; returns (ms per replay by events, ms per replay wall)."""
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


def stage_bytes(ops, H, T):
    """Algorithmic HBM bytes per launch (8 groups of one layer), averaged over layers."""
    nw = (H + 31) // 32
    route = G * F * (2 * D * 4 + 4) + G * HQ * D * 2 + G * TOPK * 12 + G * 4
    unions, avs, uniq = [], [], []
    for op in ops:
        u = op.count.cpu().numpy().astype(np.int64)
        nsel = (op.valid.cpu().numpy() > 0).sum(1)
        unions.append(int((nsel * nw * 4 + u * 4 + 4).sum() + G * TOPK * 12))
        avs.append(int(((u + T) * 2 * D * 2 + u * 4 + 4).sum() + 2 * G * HQ * D * 2))
        uniq.append(u.mean())
    return route, float(np.mean(unions)), float(np.mean(avs)), float(np.mean(uniq))


@torch.no_grad()
def update_cpu_baseline(h0, center, counts, mean, var, keys, W, b, budget_s):
    """C oracle append_index (src/prismkv/core.py:186-201) of one group's block,
    one thread: (median us, repetitions)."""
    import oracle
    oracle.build()
    index = oracle.Index(h0, center, counts, mean, var, [np.zeros(0, np.int64)] * F)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or not times:
        t0 = time.perf_counter()
        oracle.append_index(index, keys, W, b, 1.0, 8)
        times.append(time.perf_counter() - t0)
    return float(np.median(times)) * 1e6, len(times)


def update_timing(lib_path, H, blocks, steps, warmup, seed, device, cpu_budget_s=0.0):
    """Amortised index update: one prismkv_update launch sequence per replay
    (encode, BatchTopK threshold, bitmap append, moment merge for 8 groups),
    indexing a block of N keys at history H - N of a dedicated table (so the
    decode tables are untouched).  Every replay indexes the same block."""
    from prismkv_amd import Native8B
    gen = torch.Generator(device=device)
    gen.manual_seed(seed * 7919)
    out = {}
    N_max = max(blocks)
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
                        stream=torch.cuda.current_stream().cuda_stream)
        ms, _, _ = graph_time(once, steps, warmup)
        us = ms * 1e3
        flops = 2.0 * G * N * F * D
        out[str(N)] = dict(us_per_block=round(us, 2), us_per_token_per_layer=round(us / N, 4),
                           encode_gflop=round(flops / 1e9, 2), encode_tflops_if_alone=round(flops / (us * 1e-6) / 1e12, 2))
        log(f"update N={N}: {us:.1f} us per block ({us / N:.3f} us per token per layer, amortised)")
        if cpu_budget_s > 0 and N == min(blocks):
            c_us, reps = update_cpu_baseline(h0, op.center[0].cpu().numpy(), counts[0].cpu().numpy(),
                                             mean[0].cpu().numpy(), var[0].cpu().numpy(),
                                             k[0, h0:H].float().cpu().numpy(), W[0].cpu().numpy(),
                                             b[0].cpu().numpy(), cpu_budget_s)
            out[str(N)]["cpu_baseline"] = dict(
                value=round(c_us * G, 1), unit="us/block (8 groups)", cores=1, kind="port",
                sample=f"C oracle append_index of group 0's {N}-key block (encode, BatchTopK, summaries, Chan "
                       f"merge), one thread, median of {reps}; x8 for the 8 groups")
            log(f"update N={N}: CPU oracle {c_us:.0f} us for one group ({reps} repetitions)")
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
                    stream=torch.cuda.current_stream().cuda_stream)
    ms, _, _ = graph_time(once, max(2, steps // 4), max(1, warmup // 4))
    flops = 2.0 * G * H * F * D
    out = dict(history=H, ms_per_layer=round(ms, 3), groups_per_batch=op.build_batch,
               memberships_per_group=int(op.n[0].sum()), encode_gflop=round(flops / 1e9, 1),
               encode_tflops_if_alone=round(flops / (ms * 1e-3) / 1e12, 2))
    log(f"build H={H}: {ms:.2f} ms per layer (8 groups)")
    del op, k, W, b
    torch.cuda.empty_cache()
    return out


def cpu_baseline(op, q, k, v, H, budget_s, threads=1):
    """C oracle on layer 0: route + union + AV for 8 groups, on `threads`
    host threads (one group per task; the C calls release the GIL).
    Returns (median us per layer, repetitions)."""
    from concurrent.futures import ThreadPoolExecutor
    import oracle
    oracle.build()
    counts = op.n[:, :F].cpu().numpy().astype(np.int64)
    from prismkv_amd import untile_moments
    mean, var = (x.cpu().numpy() for x in untile_moments(op.moments))
    qf = q.float().cpu().numpy()
    kf = k.float().cpu().numpy()
    vf = v.float().cpu().numpy()
    bits = op.bits.cpu().numpy().view(np.uint32)
    kf = [np.ascontiguousarray(kf[g]) for g in range(G)]
    vf = [np.ascontiguousarray(vf[g]) for g in range(G)]

    def group(g):
        _, order, _, _ = oracle.bucket_scores(qf[g], counts[g], mean[g], var[g])
        feats = np.zeros(TOPK, np.int64)
        feats[:len(order)] = order
        ids = oracle.union_bits(bits[g], H, feats, (np.arange(TOPK) < len(order)).astype(np.float32))
        oracle.attend(qf[g], kf[g], vf[g], ids, H)

    times = []
    with ThreadPoolExecutor(max_workers=threads) as pool:
        t_end = time.perf_counter() + budget_s
        while time.perf_counter() < t_end or not times:
            t0 = time.perf_counter()
            if threads == 1:
                for g in range(G):
                    group(g)
            else:
                list(pool.map(group, range(G)))
            times.append(time.perf_counter() - t0)
    return float(np.median(times)) * 1e6, len(times)


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
    lib_path = _lib.DEFAULT_LIBRARY
    _lib.load(lib_path)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    stages = set(a.stages.split(","))
    H, T = a.history, a.tail
    log(f"building {a.layers} layers H={H} T={T} ...")
    t0 = time.perf_counter()
    layers = [make_layer(lib_path, i, H, T, a.seed, device) for i in range(a.layers)]
    torch.cuda.synchronize()
    log(f"built in {time.perf_counter() - t0:.1f}s; mem {torch.cuda.memory_allocated() / 2**30:.1f} GiB")

    def stream():
        return torch.cuda.current_stream().cuda_stream

    def chain():  # the decode step: Native8B.__call__ = route + attention (fused path, 1 launch per layer)
        for op, q, k, v in layers:
            op(q, k, v)

    def route_only():  # moment scoring + Top-16, one launch (Native8B.route also runs the union)
        for op, q, k, v in layers:
            op.lib.call("prismkv_route_single", q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(),
                        op.decode_work.data_ptr(), op.features.data_ptr(), op.valid.data_ptr(),
                        op.raw.data_ptr(), G, stream=stream())

    def union_only():
        for op, q, k, v in layers:
            op.lib.call("prismkv_union", op.bits.data_ptr(), op.features.data_ptr(), op.valid.data_ptr(),
                        op.union_work.data_ptr(), op.ids.data_ptr(), op.count.data_ptr(), G, op.history,
                        op.row_words, op.capacity, stream=stream())

    def attend_only():
        for op, q, k, v in layers:
            op.attention(q, k, v)

    result = {}
    chain()  # populate ids/count for the byte model and the stage graphs
    torch.cuda.synchronize()
    ms, wall, _ = graph_time(chain, a.steps, a.warmup) if "chain" in stages else (float("nan"),) * 3
    log(f"chain: {ms:.4f} ms/step events, {wall:.4f} ms/step wall")
    per_stage = {}
    if "chain" in stages:
        per_stage["decode"] = ms * 1e3 / a.layers  # one decode_kernel launch per layer
    stage_fns = (("route", route_only), ("union", union_only), ("attend", attend_only))
    for name, fn in stage_fns:
        if name in stages:
            sm, _, _ = graph_time(fn, a.steps, a.warmup)
            per_stage[name] = sm * 1e3 / a.layers
            log(f"{name}: {per_stage[name]:.2f} us/launch")
    chain()
    torch.cuda.synchronize()
    b_route, b_union, b_av, uniq = stage_bytes([l[0] for l in layers], H, T)
    nbytes = {"decode": b_route + b_union + b_av, "route": b_route, "union": b_union, "attend": b_av}
    stage_report = {}
    for name, us in per_stage.items():
        gbs = nbytes[name] / (us * 1e-6) / 1e9
        stage_report[name] = dict(us_per_launch=round(us, 3), algorithmic_bytes=int(nbytes[name]),
                                  achieved_GBps=round(gbs, 1), frac_of_peak=round(gbs / HBM_PEAK_GBS, 4))
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
    update = None
    if "update" in stages:
        blocks = [int(x) for x in a.update_blocks.split(",") if x]
        update = update_timing(lib_path, H, blocks, a.steps, a.warmup, a.seed, device,
                               cpu_budget_s=0.0 if a.no_cpu_baseline else 3.0)
    build = build_timing(lib_path, H, a.steps, a.warmup, a.seed, device) if "build" in stages else None
    fused = [n for n in ("decode",) if n in stage_report]
    dominant = max(fused or stage_report, key=lambda n: stage_report[n]["us_per_launch"]) if stage_report else None
    roofline = None
    if dominant:
        d = stage_report[dominant]
        roofline = dict(bound="hbm", achieved=d["achieved_GBps"], peak=HBM_PEAK_GBS, unit="GB/s",
                        frac=d["frac_of_peak"], traffic=measured_traffic(dominant, H, T),
                        kernel=STAGE_KERNEL.get(dominant, dominant), algorithmic_bytes=d["algorithmic_bytes"])
    cpu = None
    if not a.no_cpu_baseline:
        op, q, k, v = layers[0]
        # one host thread per KV group (the unit of parallel work), and one thread
        us_par, reps_par = cpu_baseline(op, q, k, v, H, a.cpu_seconds / 2, threads=G)
        us_one, reps_one = cpu_baseline(op, q, k, v, H, a.cpu_seconds / 2, threads=1)
        cpu = dict(value=round(us_par, 1), unit="us/layer", cores=G, kind="port",
                   sample=f"layer 0 of the workload (8 groups, H={H}, T={T}): C oracle route + union + AV, "
                          f"one group per host thread, median of {reps_par} repetitions; single thread: "
                          f"{us_one:.1f} us/layer (median of {reps_one})",
                   value_1_thread=round(us_one, 1))
    value = ms * 1e3 / a.layers
    result = {
        "metric": METRIC, "value": round(value, 3), "unit": "us/layer", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": round(value / PPU_US_PER_LAYER_64K, 4), "dtype": "fp32", "data": "synthetic",
        "config": {"workload": f"8B-geometry routed decode, {a.layers} layers x 8 KV groups x 4 Q heads, d=128, "
                               f"F=3000, Top-16, H={H} + {T} tail, bf16 KV, per-key top-8 SAE membership",
                   "layers": a.layers, "groups": G, "history": H, "tail": T,
                   "kv_dtype": "bf16", "mean_unique_ids_per_group": round(uniq, 1), "parallelism": "single GPU"},
        "wall_ms_per_step": round(wall, 4), "stages": stage_report, "copy_probe_GBps": copy_gbs and round(copy_gbs, 1),
        "update": update, "build": build, "roofline": roofline, "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
