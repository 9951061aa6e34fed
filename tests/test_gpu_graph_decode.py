"""Decode steps replayed from a HIP graph while the tail grows.

  * `Native8B.__call__(..., tail=t)` (`prismkv_decode_tail`: the tail length
    read from device memory at launch) gives bit-identical features, ids,
    counts and output to the host-length launch over the same rows;
  * one captured launch replayed with different device tail lengths equals
    the eager launch for each;
  * `hf.DecodeGraph`: a small random-init Qwen3 with the 8B attention
    geometry decodes from a transformers StaticCache; the eager steps match
    the oracle's route + attention (src/prismkv/core.py:106-183) over the
    index the device holds, the update policy (hf_reference.py:205-211)
    moves the history across the run, and the graph-replayed steps give
    bit-identical logits to the eager ones and the same records (read back
    from the per-step device ring) as the eager steps' operators held.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import cases
from tests.gpu_util import bf16_bits, log, operator, route_outputs
from tests.test_gpu_hf import Capture, check_call, encoders, tiny_qwen3

pytestmark = pytest.mark.gpu


def _snapshot(op):
    return [bf16_bits(op.out).copy(), *[x.copy() for x in route_outputs(op)]]


def _same(a, b):
    return all(np.array_equal(x, y) for x, y in zip(a, b))


def test_device_tail_matches_host_tail():
    case = cases.native_case(4096, 64, "random", seed=4)
    op, q, k, v = operator(case)
    H = op.history
    t = torch.zeros(1, dtype=torch.int32, device="cuda")
    for T in (0, 1, 37, 64):
        op(q, k[:, :H + T], v[:, :H + T])
        torch.cuda.synchronize()
        host = _snapshot(op)
        op.out.zero_()
        op.ids.zero_()
        t.fill_(T)
        op(q, k, v, tail=t)
        torch.cuda.synchronize()
        assert _same(host, _snapshot(op)), T
    # a word beyond K's rows is clamped to them
    t.fill_(1000)
    op(q, k, v, tail=t)
    torch.cuda.synchronize()
    assert _same(host, _snapshot(op))
    assert op.decode_errors() == 0


def test_captured_launch_follows_the_tail_word():
    case = cases.native_case(8192, 256, "random", seed=6)
    op, q, k, v = operator(case)
    H = op.history
    want = {}
    for T in (256, 1, 100, 0, 255):
        op(q, k[:, :H + T], v[:, :H + T])
        torch.cuda.synchronize()
        want[T] = _snapshot(op)
    t = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        op(q, k, v, tail=t)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        op(q, k, v, tail=t)
    for T in (256, 1, 100, 0, 255):
        op.out.zero_()
        t.fill_(T)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert _same(want[T], _snapshot(op)), T
    assert op.decode_errors() == 0


def _prefill(session, model, cache, ids, P, chunk=1024):
    with torch.no_grad(), session.prefill():
        for lo in range(0, P, chunk):
            hi = min(P, lo + chunk)
            model(ids[:, lo:hi], position_ids=torch.arange(lo, hi, device="cuda")[None], past_key_values=cache,
                  use_cache=True, logits_to_keep=1)


def test_static_cache_decode_graph():
    from transformers import StaticCache
    from prismkv_amd.hf import DecodeGraph, HFNative
    layers, P, N, interval = 2, 2048, 80, 64
    model = tiny_qwen3(layers)
    session = HFNative(model, encoders(layers), update_interval=interval)
    ids = torch.randint(0, 256, (1, P + N), generator=torch.Generator().manual_seed(9)).cuda()
    logits, records, expected = {}, {}, []
    checks = {0, 64, N - 1}
    for use_graph in (False, True):
        session.begin_request()
        cache = StaticCache(config=model.config, max_cache_len=P + N + 16)
        # a 32-step record ring: read back twice during the run and once at the end
        step = DecodeGraph(session, cache, graph=use_graph, record_steps=32)
        _prefill(session, model, cache, ids, P)
        cap = Capture(session) if not use_graph else None
        out = []
        for s in range(N):
            n_calls = len(cap.calls) if cap else 0
            out.append(step(ids[:, P + s:P + s + 1]).clone())
            if cap:  # the records each eager step must leave, read from the operators
                torch.cuda.synchronize()
                for layer in sorted(session.ops):
                    op = session.ops[layer]
                    for g, (u, r, b) in enumerate(zip(op.count.tolist(), op.raw.tolist(),
                                                      (op.valid > 0).sum(1).tolist())):
                        expected.append(dict(layer=layer, group=g, history=op.history, unique=u, raw=r, buckets=b,
                                             tail=P + s + 1 - op.history, routing_policy="sparse"))
            if cap and s in checks:
                torch.cuda.synchronize()
                for layer, q, K, V, o in cap.calls[n_calls:]:
                    total = P + s + 1
                    err = check_call(session.ops[layer], layer, q, K[:, :total], V[:, :total], o)
                    log(f"  eager step {s} layer {layer}: history={session.ops[layer].history} {err}")
            if cap:
                cap.calls = []
        torch.cuda.synchronize()
        if cap:
            session.forward = cap._forward
        for layer, op in session.ops.items():
            assert op.history == P + interval, (use_graph, layer, op.history)
            assert op.decode_errors() == 0
        step.close()
        logits[use_graph] = torch.stack(out)
        records[use_graph] = [dict(r) for r in session.records]
        log(f"graph={use_graph}: {N} steps, histories {[op.history for op in session.ops.values()]}")
    assert torch.isfinite(logits[False]).all()
    assert torch.equal(logits[False], logits[True])
    assert len(expected) == N * layers * 8
    assert records[False] == expected
    assert records[True] == expected
    session.close()


def test_36_layer_step_graph():
    # the 36 attention layers of the 8B geometry (32 query / 8 KV heads,
    # d = 128; hidden 1024 keeps the random weights small): the whole
    # one-token forward captured once and replayed, bit-identical to eager
    import time
    from transformers import Qwen3Config, Qwen3ForCausalLM, StaticCache
    from prismkv_amd.hf import DecodeGraph, HFNative
    L, P, N = 36, 8192, 8
    cfg = Qwen3Config(vocab_size=1000, hidden_size=1024, intermediate_size=2048, num_hidden_layers=L,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=16384)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(5)
    model = Qwen3ForCausalLM(cfg).to(device="cuda", dtype=torch.bfloat16).eval()
    session = HFNative(model, encoders(L))
    ids = torch.randint(0, 1000, (1, P + N), generator=torch.Generator().manual_seed(12)).cuda()
    logits, ms = {}, {}
    for use_graph in (False, True):
        session.begin_request()
        cache = StaticCache(config=cfg, max_cache_len=P + N + 8)
        step = DecodeGraph(session, cache, graph=use_graph)
        _prefill(session, model, cache, ids, P, chunk=2048)
        out, times = [], []
        for s in range(N):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out.append(step(ids[:, P + s:P + s + 1]).clone())
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        assert all(op.decode_errors() == 0 and op.history == P for op in session.ops.values())
        if use_graph:
            unique = [float(session.ops[layer].count.float().mean()) for layer in sorted(session.ops)]
            log("  unique ids per group by layer (last step): " + " ".join(f"{u:.0f}" for u in unique))
        step.close()
        logits[use_graph] = torch.stack(out)
        ms[use_graph] = 1e3 * float(np.median(times[2:]))
    log(f"36-layer one-token step, H={P}: eager {ms[False]:.2f} ms, graph replay {ms[True]:.2f} ms")
    assert torch.isfinite(logits[False]).all()
    assert torch.equal(logits[False], logits[True])
    session.close()


def test_static_cache_decode_graph_with_cap():
    # DecodeGraph over the capped step (route, budgeted walk, union + attention
    # with the device tail length): replays bit-identical to the eager steps,
    # and the eager steps match the oracle's walk over the device's index
    from transformers import StaticCache
    from prismkv_amd.hf import DecodeGraph, HFNative
    layers, P, N, interval, cap = 2, 2048, 40, 32, 0.05
    model = tiny_qwen3(layers)
    session = HFNative(model, encoders(layers, seed=31), update_interval=interval, unique_cap=cap)
    ids = torch.randint(0, 256, (1, P + N), generator=torch.Generator().manual_seed(19)).cuda()
    logits = {}
    for use_graph in (False, True):
        session.begin_request()
        cache = StaticCache(config=model.config, max_cache_len=P + N + 16)
        step = DecodeGraph(session, cache, graph=use_graph)
        _prefill(session, model, cache, ids, P)
        out = []
        for s in range(N):
            out.append(step(ids[:, P + s:P + s + 1]).clone())
            if not use_graph and s in (0, N - 1):
                torch.cuda.synchronize()
                for layer, op in session.ops.items():
                    got = op.export_indices()
                    feats, valid = op.features.cpu().numpy(), op.valid.cpu().numpy()
                    count = op.count.cpu().numpy()
                    for g in range(8):
                        kept = [int(f) for f, ok in zip(feats[g], valid[g]) if ok > 0]
                        lists = [l.numpy() for l in got[g].lists]
                        w_ids, meta = oracle.select_buckets(np.array(kept, np.int64), lists, op.history, None)
                        assert len(w_ids) <= int(op.history * cap)
                        assert np.array_equal(op.ids[g, :count[g]].cpu().numpy().astype(np.int64), w_ids)
                        assert int(op.raw[g]) == meta["raw"]
        torch.cuda.synchronize()
        for op in session.ops.values():
            assert op.decode_errors() == 0
        step.close()
        logits[use_graph] = torch.stack(out)
        log(f"capped graph={use_graph}: {N} steps, histories {[op.history for op in session.ops.values()]}, "
            f"unique {[int(op.count.max()) for op in session.ops.values()]}")
    assert torch.isfinite(logits[False]).all()
    assert torch.equal(logits[False], logits[True])
    session.close()
