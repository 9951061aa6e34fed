"""GPU parity of the MI355X decode path against the CPU oracle.

Bucket features (rank order), raw, unique IDs and counts must be identical;
the attention output must be within relative L2 2e-3 of the fp64 oracle (and
max-abs < 0.05, the reference witness bound, examples/check_native8b.py:55-61).
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import cases, expect
from prismkv_amd._lib import nbytes
from tests.gpu_util import bf16_bits, device_layer, log, operator, route_outputs

pytestmark = pytest.mark.gpu

AV_TOL = 2e-3


def check_case(case, splits_list=(32, 64, 128), schedules=(0, 2)):
    log(f"case kind={case['kind']} H={case['H']} T={case['T']}")
    op, q, k, v = operator(case)
    op.route(q)
    groups = expect.expected(case)
    identical, near = expect.compare_route(groups, *route_outputs(op))
    margins = ["%.2e" % g["margin"] for g in groups]
    log(f"  route: {identical} groups identical to the oracle order, {near} differ only at near-ties; "
        f"unique={[len(g['ids']) for g in groups]} margins={margins}")
    assert identical + near == len(groups)
    want = expect.expected_attention(case, groups)
    for splits in splits_list:
        for schedule in schedules:
            out = op.attention(q, k, v, splits=splits, schedule=schedule)
            torch.cuda.synchronize()
            err = expect.attention_errors(bf16_bits(out), want)
            log(f"  splits={splits} schedule={schedule} {err}")
            assert np.isfinite(bf16_bits(out).astype(np.float32)).all()
            assert err["rel_l2"] <= AV_TOL and err["max_abs"] < 0.05, err
    # the fused decode path (Native8B.__call__) gives the same selection and ids
    features, valid, raw, ids, count = route_outputs(op)
    out = op(q, k, v)
    torch.cuda.synchronize()
    f2, v2, r2, i2, c2 = route_outputs(op)
    assert np.array_equal(features, f2) and np.array_equal(valid, v2) and np.array_equal(raw, r2)
    assert np.array_equal(count, c2)
    for g in range(8):
        assert np.array_equal(ids[g][:count[g]], i2[g][:c2[g]]), ("fused ids", g)
    err = expect.attention_errors(bf16_bits(out), want)
    log(f"  fused decode {err}")
    assert err["rel_l2"] <= AV_TOL and err["max_abs"] < 0.05, err
    # no bounded inter-workgroup wait of the single-launch decode gave up
    assert op.decode_errors() == 0
    return op, groups


@pytest.mark.parametrize("H,tail,kind", cases.NATIVE_CASES)
def test_native_witness_cases(H, tail, kind):
    # examples/check_native8b.py:80 -- the reference's six synthetic cases
    op, groups = check_case(cases.native_case(H, tail, kind))
    if kind in ("ties", "few", "empty"):
        # reviewer_guide/native8b_validation.json unique counts (RNG independent)
        assert op.count.cpu().tolist() == [{"ties": 16, "few": 65, "empty": 0}[kind]] * 8


def test_replay_shape_global_budget_index():
    # examples/replay.py shape, index built with the reference BatchTopK rule
    check_case(cases.replay_case(seed=5), splits_list=(64,), schedules=(0,))


def test_8b_geometry_64k_topk8():
    # 8 groups x 4 heads, d=128, F=3000, H=65536 + 256 tail, per-key top-8 membership
    check_case(cases.topk8_case(H=65536, T=256, seed=2), splits_list=(16, 64, 128), schedules=(0,))


def test_8b_geometry_64k_long_tail():
    # the update policy leaves tails of up to 4096 rows between index updates
    # (configs/submitted_8b.json:14).  2100 rows are 66 per workgroup at 32
    # workgroups per group: the fused decode requests each wave's first tail
    # block early (16 rows for waves 0-3, 2 for wave 4, none for waves 5-7)
    # and attends it in a slot of the wave's first round
    check_case(cases.topk8_case(H=65536, T=2100, seed=3), splits_list=(64,), schedules=(0,))


def adversarial_case(name, H=4096, T=40, seed=11):
    rng = np.random.default_rng(seed)
    k = cases.bf16_normal((seed, 0), (8, H + T, 128))
    v = cases.bf16_normal((seed, 1), (8, H + T, 128))
    q = cases.bf16_normal((seed, 2), (8, 4, 128))
    from oracle import Index
    indices = []
    for g in range(8):
        counts = np.ones(3000, np.int64)
        mean = np.zeros((3000, 128), np.float32)
        var = np.zeros((3000, 128), np.float32)
        if name == "empty":
            counts[:] = 0
        elif name == "fewer_than_16":
            counts[13:] = 0
        elif name == "count_steps":          # near-ties and exact ties in the count term only
            counts = 1 + rng.permutation(3000) // 10
        elif name in ("masked_random", "large_range"):
            counts = rng.integers(0, 150, 3000)
            counts[::3] = 0
            std = 2.0 if name == "large_range" else 0.3
            mean = (rng.standard_normal((3000, 128)) * std / np.sqrt(128) * 4).astype(np.float32)
            var = (rng.random((3000, 128)) * std).astype(np.float32)
        lists = [np.sort(rng.choice(H, min(int(c), H), replace=False)) for c in counts]
        indices.append(Index(H, np.zeros(128, np.float32), counts, mean, var, lists))
    return dict(H=H, T=T, q=q, k=k, v=v, indices=indices, kind=name)


@pytest.mark.parametrize("name", ["empty", "fewer_than_16", "all_equal", "count_steps", "masked_random",
                                  "large_range"])
def test_adversarial_top16(name):
    # kernels/cuda_sm90/benchmark_hopper_route.py:62-75 patterns, adapted to moments input
    check_case(adversarial_case(name), splits_list=(64,), schedules=(0,))


def test_repeat_calls_are_bitwise_identical():
    case = cases.native_case(1025, 3, "random")
    op, q, k, v = operator(case)
    outs = []
    for _ in range(3):
        out = op(q, k, v, splits=32).clone()
        outs.append((bf16_bits(out), *[x.copy() for x in route_outputs(op)]))
    for o in outs[1:]:
        for a, b in zip(outs[0], o):
            assert np.array_equal(a, b)


def test_graph_replay_matches_eager():
    # the decode step allocates nothing and never syncs: capture it and replay
    case = cases.native_case(1025, 3, "random")
    op, q, k, v = operator(case)
    eager = bf16_bits(op(q, k, v, splits=64).clone())
    eager_ids = op.ids.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        op(q, k, v, splits=64)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        op(q, k, v, splits=64)
    for i in range(4):
        op.out.zero_()
        op.ids.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(op.out), eager), i
        assert torch.equal(op.ids, eager_ids), i
        _ = (torch.randn(1000, device="cuda") * 2).sum().item()   # unrelated eager work between replays


def test_no_tail_and_uneven_split_count():
    # T = 0 (the step right after an index update) and H = 81920: 80-word union
    # tiles, two 64-word chunks per workgroup
    check_case(cases.native_case(4096, 0, "random", seed=7), splits_list=(32,), schedules=(0,))
    check_case(cases.native_case(81920, 9, "random", seed=8), splits_list=(64,), schedules=(0,))


def test_long_history_uses_split_path(monkeypatch):
    # beyond the single-launch limit Native8B.__call__ runs route + attention;
    # the limit is lowered here so a small case takes that branch
    import prismkv_amd.native8b as nb
    monkeypatch.setattr(nb, "FUSED_MAX_HISTORY", 1000)
    check_case(cases.native_case(1025, 3, "random"), splits_list=(32,), schedules=(0,))


def test_fused_decode_long_tiles():
    # H = 300000: 293-word union tiles (5 chunks, 9376 tokens per workgroup)
    check_case(cases.native_case(300000, 3, "random", seed=9), splits_list=(128,), schedules=(0,))


def test_fused_decode_one_word_second_chunk():
    # H = 65537: 65-word union tiles, the second chunk of each one word long
    check_case(cases.native_case(65537, 5, "ties", seed=21), splits_list=(64,), schedules=(0,))


def test_fused_decode_largest_history_matches_split_path():
    # H = 524288, the single launch's limit: 512-word tiles (8 chunks, 16384
    # tokens and 64 KB of row list per workgroup).  The oracle's case
    # generator is too slow at this size, so the layer is built on the device
    # and the single launch must select exactly what the separate route +
    # union select (oracle-checked up to H = 300000) and attend within the
    # same tolerance
    op, q, k, v = device_layer(524288, 7, seed=3)
    fused = bf16_bits(op(q, k, v).clone())
    f1 = route_outputs(op)
    op.route(q)
    split = bf16_bits(op.attention(q, k, v).clone())
    f2 = route_outputs(op)
    for a, b in zip(f1[:3], f2[:3]):
        assert np.array_equal(a, b)
    assert np.array_equal(f1[4], f2[4])
    for g in range(8):
        assert np.array_equal(f1[3][g][:f1[4][g]], f2[3][g][:f2[4][g]]), g
    rel = np.linalg.norm(oracle.bf16_to_f32(fused).astype(np.float64) - oracle.bf16_to_f32(split)) / \
        np.linalg.norm(oracle.bf16_to_f32(split).astype(np.float64))
    log(f"  H=524288: unique ids per group {f1[4].tolist()}, fused vs split relL2 {rel:.2e}")
    assert rel <= AV_TOL and op.decode_errors() == 0


@pytest.mark.parametrize("H", [4096, 65536])
def test_single_launch_route_matches_three_launch_route(H):
    # prismkv_route_single (one launch, the decode's selection phases, on the
    # decode workspace) against prismkv_route (scoring, parts, final): the same
    # features, valid and raw bits, on repeated calls and after a decode on
    # the same workspace (each launch leaves the workspace zero)
    op, q, k, v = device_layer(H, 16, seed=11)
    lib, s = op.lib, torch.cuda.current_stream().cuda_stream
    work = torch.zeros(lib.query("prismkv_route_work_bytes", 8), dtype=torch.uint8, device="cuda")

    def three():
        lib.call("prismkv_route", q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(), work.data_ptr(),
                 op.features.data_ptr(), op.valid.data_ptr(), op.raw.data_ptr(), 8, nbytes(work), stream=s)

    def one():
        lib.call("prismkv_route_single", q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(),
                 op.decode_work.data_ptr(), op.features.data_ptr(), op.valid.data_ptr(), op.raw.data_ptr(), 8,
                 nbytes(op.decode_work), stream=s)

    def selection():
        torch.cuda.synchronize()
        out = [x.cpu().numpy().copy() for x in (op.features, op.valid, op.raw)]
        for x in (op.features, op.valid, op.raw):
            x.zero_()
        return out

    three()
    want = selection()
    for step in range(3):
        one()
        got = selection()
        for a, b in zip(want, got):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), step
        if step == 1:
            op(q, k, v)
            torch.cuda.synchronize()
    assert int(op.decode_work.view(torch.int32)[0]) == 0
    log(f"  H={H}: single-launch route equals the three-launch route over 3 calls; "
        f"buckets of group 0: {want[0][0].tolist()}")


def test_union_262k_history():
    # H beyond the reference union limit (131072): 8 groups x 262144 tokens
    check_case(cases.native_case(262144, 64, "random", seed=5), splits_list=(128,), schedules=(0,))


@pytest.mark.parametrize("H,tail,kind,cap", [(65, 7, "few", 0.3), (1025, 3, "random", 0.01),
                                             (65536, 17, "random", 0.002), (262144, 5, "random", 0.01),
                                             (300000, 7, "random", 0.005)])
def test_strict_unique_cap(H, tail, kind, cap):
    # src/prismkv/core.py:149-163: with a cap, a ranked bucket whose new ids would
    # push the union past floor(H * cap) is skipped and the walk goes on.  The
    # device's own ranked order (checked against the oracle first) is fed to the
    # oracle's select_buckets, so the budgeted walk is checked bit-exactly.
    # The three walk variants: up to 2048 bitmap words (H <= 65536), up to 8192
    # (H = 262144, the stress history) and the LDS-union one (H = 300000).
    case = cases.native_case(H, tail, kind)
    log(f"cap case kind={kind} H={H} T={tail} cap={cap}")
    op, q, k, v = operator(case)
    op.route(q)
    groups = expect.expected(case)
    identical, near = expect.compare_route(groups, *route_outputs(op))
    assert identical + near == 8
    features, valid, _, _, _ = route_outputs(op)
    orders = [features[g][valid[g] > 0] for g in range(8)]
    op.unique_cap = cap
    op.route(q)
    f2, v2, r2, i2, c2 = route_outputs(op)
    want = []
    skipped = 0
    for g in range(8):
        ids, meta = oracle.select_buckets(orders[g], case["indices"][g].lists, H, cap)
        nf = len(meta["features"])
        skipped += len(orders[g]) - nf
        assert f2[g][:nf].tolist() == meta["features"], ("kept buckets", g)
        assert not f2[g][nf:].any() and v2[g].tolist() == [1.0] * nf + [0.0] * (16 - nf), ("padding", g)
        assert int(r2[g]) == meta["raw"] and int(c2[g]) == len(ids) <= meta["limit"], ("raw/count", g)
        assert np.array_equal(i2[g][:len(ids)].astype(np.int64), ids), ("ids", g)
        want.append(dict(ids=ids))
    log(f"  {skipped} ranked buckets skipped by the budget across 8 groups")
    expected = expect.expected_attention(case, want)
    out = op.attention(q, k, v)
    torch.cuda.synchronize()
    first = bf16_bits(out).copy()
    err = expect.attention_errors(first, expected)
    assert err["rel_l2"] <= AV_TOL and err["max_abs"] < 0.05, err
    # __call__ with a cap: route, the walk spread over the group's
    # workgroups, union and attention in one launch (prismkv_decode_capped):
    # the same selection, ids and count, and the attention within the bound
    op.ids.zero_()
    op.count.zero_()
    out = op(q, k, v)
    torch.cuda.synchronize()
    f3, v3, r3, i3, c3 = route_outputs(op)
    for a, b in ((f2, f3), (v2, v3), (r2, r3), (c2, c3)):
        assert np.array_equal(a, b)
    for g in range(8):
        assert np.array_equal(i3[g][:c3[g]], i2[g][:c2[g]]), ("ids, one launch", g)
    err = expect.attention_errors(bf16_bits(out), expected)
    log(f"  capped call, one launch: {err}")
    assert err["rel_l2"] <= AV_TOL and err["max_abs"] < 0.05, err
    # ... and the three launches (route, prismkv_select_cap,
    # prismkv_union_attend over the walked selection): the same rows, attended
    # in another order (the one launch takes each window's rows as the walk
    # decides them), so the outputs agree to rounding
    fused = bf16_bits(out).copy()
    three = three_launch_capped(op, q, k, v)
    assert same_rows_close(fused, three), "capped: one launch vs three"
    assert op.decode_errors() == 0


def same_rows_close(a_bits, b_bits, tol=1e-3):
    """Two bf16 outputs of attention over the same rows in different orders:
    within `tol` relative L2 (fp32 accumulation order, then bf16 rounding)."""
    a = oracle.bf16_to_f32(a_bits).astype(np.float64)
    b = oracle.bf16_to_f32(b_bits).astype(np.float64)
    return oracle.rel_l2(a, b) <= tol


def three_launch_capped(op, q, k, v, groups=8, work=None):
    """The capped step as three launches into op's buffers: the route
    (prismkv_route_single), the walk (prismkv_select_cap) and union +
    attention over the walked selection (prismkv_union_attend); out bits."""
    s = torch.cuda.current_stream().cuda_stream
    work = op.decode_work if work is None else work
    op.lib.call("prismkv_route_single", q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(), work.data_ptr(),
                op.features.data_ptr(), op.valid.data_ptr(), op.raw.data_ptr(), groups, nbytes(work), stream=s)
    op.lib.call("prismkv_select_cap", op.bits.data_ptr(), op.n.data_ptr(), op.features.data_ptr(),
                op.valid.data_ptr(), op.raw.data_ptr(), groups, op.history, op._cap_limit(), op.row_words, stream=s)
    op.lib.call("prismkv_union_attend", q.data_ptr(), op.bits.data_ptr(), k.data_ptr(), v.data_ptr(),
                work.data_ptr(), op.features.data_ptr(), op.valid.data_ptr(), op.ids.data_ptr(),
                op.count.data_ptr(), op.out.data_ptr(), groups, op.history, k.shape[1] - op.history, op.capacity,
                op.row_words, k.stride(0), v.stride(0), op.capacity, nbytes(work), stream=s)
    torch.cuda.synchronize()
    return bf16_bits(op.out).copy()


@pytest.mark.parametrize("H,pad", [(1000, 0), (65536, 0), (65536, 1), (100000, 0), (262144, 0), (200000, 1),
                                   (300000, 0)])
def test_cap_walk_layouts(H, pad):
    # prismkv_select_cap straight on bitmaps (src/prismkv/core.py:149-163):
    # 16-byte runs at up to 2048 / 4096 / 8192 words a row (the latter two
    # with row-touching workgroups), single words where a row is not 16-byte
    # aligned (pad = 1 makes row_words odd), the LDS-union walk above 8192
    # words or for an odd layout above 2048.  Rows of densities 1/2 .. 1/64,
    # a selection with gaps and an out-of-range id, limits that keep from
    # none to most of the ranked buckets; features / valid / raw must equal
    # the oracle's walk over the valid ranked buckets.
    from prismkv_amd import _lib
    lib = _lib.load()
    G, F = 8, 3000
    nw = (H + 31) // 32
    row_words = nw + pad
    rng = np.random.default_rng(H + pad)
    bits = torch.zeros(G, F, row_words, dtype=torch.int32, device="cuda")
    counts = torch.zeros(G, 3008, dtype=torch.int32, device="cuda")
    sel = np.stack([rng.permutation(F)[:16] for _ in range(G)]).astype(np.int64)
    valid = np.ones((G, 16), np.float32)
    valid[:, 5] = 0.0       # a gap in the ranked list
    sel[3, 9] = F + 7       # an out-of-range id selects nothing
    lists = [dict() for _ in range(G)]
    for g in range(G):
        for j in range(16):
            b = int(sel[g, j])
            if b >= F:
                continue
            dens = 2.0 ** -rng.integers(1, 7)
            member = np.flatnonzero(rng.random(H) < dens)
            lists[g][b] = member
            words = np.zeros(row_words, np.uint32)
            np.bitwise_or.at(words, member >> 5, (np.uint32(1) << (member & 31).astype(np.uint32)))
            bits[g, b] = torch.from_numpy(words.view(np.int32)).cuda()
            counts[g, b] = len(member)
    stream = torch.cuda.current_stream().cuda_stream
    for cap in (1 / 64, 1 / 16, 1 / 5, 1.0):
        f = torch.from_numpy(sel).cuda()
        v = torch.from_numpy(valid).cuda()
        raw = torch.zeros(G, dtype=torch.int32, device="cuda")
        limit = int(np.floor(H * cap))
        lib.call("prismkv_select_cap", bits.data_ptr(), counts.data_ptr(), f.data_ptr(), v.data_ptr(), raw.data_ptr(),
                 G, H, limit, row_words, stream=stream)
        torch.cuda.synchronize()
        f, v, raw = f.cpu().numpy(), v.cpu().numpy(), raw.cpu().numpy()
        kept = []
        for g in range(G):
            order = [int(b) for b, ok in zip(sel[g], valid[g]) if ok > 0 and b < F]
            table = [lists[g].get(b, np.zeros(0, np.int64)) for b in range(F)]
            _, meta = oracle.select_buckets(np.array(order, np.int64), table, H, cap)
            nf = len(meta["features"])
            assert meta["limit"] == limit
            assert f[g][:nf].tolist() == meta["features"] and not f[g][nf:].any(), (cap, g)
            assert v[g].tolist() == [1.0] * nf + [0.0] * (16 - nf), (cap, g)
            assert int(raw[g]) == meta["raw"], (cap, g)
            kept.append(nf)
        log(f"  walk H={H} row_words={row_words} cap={cap:.4f}: kept {kept}")


@pytest.mark.parametrize("groups", [1, 2, 3, 4, 6, 8])
def test_capped_decode_groups(groups):
    # prismkv_decode_capped on the first `groups` groups (32 .. 256 workgroups
    # per group, so 32 .. 256 records per walk window): features / valid /
    # raw / ids / count bit for bit as the three launches on the same groups,
    # and out to rounding (the same rows in window order), at caps that keep
    # from none to all of the ranked buckets
    case = cases.native_case(32768, 40, "random", seed=17)
    op, q, k, v = operator(case)
    s = torch.cuda.current_stream().cuda_stream
    work = torch.zeros(op.lib.query("prismkv_decode_work_bytes", groups, op.capacity), dtype=torch.uint8,
                       device="cuda")
    kept = []
    for cap in (0.0, 0.01, 0.05, 0.2, 1.0):
        op.unique_cap = cap
        three = three_launch_capped(op, q, k, v, groups, work)
        ref = [x.clone() for x in (op.features, op.valid, op.raw, op.ids, op.count)]
        for x in (op.features, op.valid, op.raw, op.ids, op.count, op.out):
            x.zero_()
        op.lib.call("prismkv_decode_capped", q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(),
                    op.bits.data_ptr(), k.data_ptr(), v.data_ptr(), work.data_ptr(), op.features.data_ptr(),
                    op.valid.data_ptr(), op.raw.data_ptr(), op.ids.data_ptr(), op.count.data_ptr(),
                    op.out.data_ptr(), groups, op.history, k.shape[1] - op.history, op.capacity, op._cap_limit(),
                    op.row_words, k.stride(0), v.stride(0), op.capacity, nbytes(work), stream=s)
        torch.cuda.synchronize()
        assert int(work[:4].view(torch.int32)[0]) == 0  # no bounded wait gave up
        got = (op.features, op.valid, op.raw, op.ids, op.count)
        for g in range(groups):
            for a, b in zip(got[:3], ref[:3]):
                assert torch.equal(a[g], b[g]), (cap, g)
            n = int(ref[4][g])
            assert int(got[4][g]) == n and torch.equal(got[3][g][:n], ref[3][g][:n]), (cap, g)
        assert same_rows_close(bf16_bits(op.out)[:groups], three[:groups]), cap
        kept.append([int((op.valid[g] > 0).sum()) for g in range(groups)])
    log(f"  groups={groups}: kept buckets per cap {kept}")


@pytest.mark.parametrize("groups", [1, 2, 3, 5, 7])
def test_route_union_fewer_groups(groups):
    # prismkv_route_union on the first `groups` groups runs 256 / groups
    # workgroups per group (64 .. 256: count slots of 64 .. 256 readers, each
    # reader polling up to 4 chunks of 64 lower tiles); it selects and lists
    # exactly what the 8-group launch does for those groups, twice in a row
    # on one workspace, which it leaves zero
    op, q, k, v = device_layer(16384, 16, seed=21)
    s = torch.cuda.current_stream().cuda_stream
    op.route(q)
    torch.cuda.synchronize()
    want = route_outputs(op)
    work = torch.zeros(op.lib.query("prismkv_decode_work_bytes", groups, op.capacity), dtype=torch.uint8,
                       device="cuda")
    for call in range(2):
        feats, valid, raw = torch.zeros_like(op.features), torch.zeros_like(op.valid), torch.zeros_like(op.raw)
        ids, count = torch.zeros_like(op.ids), torch.zeros_like(op.count)
        op.lib.call("prismkv_route_union", q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(), op.bits.data_ptr(),
                    work.data_ptr(), feats.data_ptr(), valid.data_ptr(), raw.data_ptr(), ids.data_ptr(),
                    count.data_ptr(), groups, op.history, op.capacity, op.row_words, op.capacity, nbytes(work),
                    stream=s)
        torch.cuda.synchronize()
        assert int(work[:4].view(torch.int32)[0]) == 0  # no bounded wait gave up
        got = (feats.cpu().numpy(), valid.cpu().numpy(), raw.cpu().numpy(), ids.cpu().numpy(), count.cpu().numpy())
        for g in range(groups):
            assert np.array_equal(got[0][g], want[0][g]) and np.array_equal(got[1][g], want[1][g]), (call, g)
            assert got[2][g] == want[2][g] and got[4][g] == want[4][g], (call, g)
            assert np.array_equal(got[3][g][:got[4][g]], want[3][g][:want[4][g]]), (call, g)
        assert not bool(work[16:].any()), "the workspace is left zero"
    log(f"  groups={groups}: route_union equals the 8-group launch, unique ids {got[4][:groups].tolist()}")


def test_capped_decode_unaligned_rows():
    # prismkv_decode_capped reads the walk's words 4 a lane when every bucket
    # row is 16-byte aligned (row_words a multiple of 4, as Native8B lays the
    # bitmaps out) and one word a thread otherwise: the same bitmaps with one
    # padding word a row (odd row_words) give bit-identical outputs
    case = cases.native_case(32768, 40, "random", seed=19)
    op, q, k, v = operator(case)
    s = torch.cuda.current_stream().cuda_stream
    groups = 8
    work = torch.zeros(op.lib.query("prismkv_decode_work_bytes", groups, op.capacity), dtype=torch.uint8,
                       device="cuda")
    padded = torch.zeros(op.bits.shape[0], op.bits.shape[1], op.row_words + 1, dtype=op.bits.dtype, device="cuda")
    padded[:, :, :op.row_words] = op.bits
    assert op.row_words % 4 == 0 and (op.row_words + 1) % 4 != 0
    for cap in (0.01, 0.05, 1.0):
        op.unique_cap = cap
        outs = []
        for bits, rw in ((op.bits, op.row_words), (padded, op.row_words + 1)):
            for x in (op.features, op.valid, op.raw, op.ids, op.count, op.out):
                x.zero_()
            op.lib.call("prismkv_decode_capped", q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(),
                        bits.data_ptr(), k.data_ptr(), v.data_ptr(), work.data_ptr(), op.features.data_ptr(),
                        op.valid.data_ptr(), op.raw.data_ptr(), op.ids.data_ptr(), op.count.data_ptr(),
                        op.out.data_ptr(), groups, op.history, k.shape[1] - op.history, op.capacity,
                        op._cap_limit(), rw, k.stride(0), v.stride(0), op.capacity, nbytes(work), stream=s)
            torch.cuda.synchronize()
            assert int(work[:4].view(torch.int32)[0]) == 0  # no bounded wait gave up
            outs.append([x.clone() for x in (op.features, op.valid, op.raw, op.ids, op.count, op.out)])
        for a, b in zip(*outs):
            assert torch.equal(a, b), cap
        log(f"  cap={cap}: aligned and odd row_words identical, unique ids {outs[0][4].tolist()}")


@pytest.mark.parametrize("groups", [1, 2, 3, 4, 5, 7])
def test_fused_decode_fewer_groups(groups):
    # prismkv_decode on the first `groups` groups runs 256 / groups workgroups
    # per group (64 / 128 / 256 splits: 2, 4 or 8 candidate sets per wave in
    # the selection; 85, 51 and 36 splits leave the last set partly empty); it
    # selects exactly what the 8-group launch selects for those groups, and
    # its attention is within tolerance of the oracle's
    case = cases.native_case(16384, 40, "random", seed=13)
    op, q, k, v = operator(case)
    op(q, k, v)
    torch.cuda.synchronize()
    ref = route_outputs(op)
    groups_want = expect.expected(case)
    want = expect.expected_attention(case, groups_want)
    work = torch.zeros(op.lib.query("prismkv_decode_work_bytes", groups, op.capacity), dtype=torch.uint8,
                       device="cuda")
    feats, valid, raw = torch.zeros_like(op.features), torch.zeros_like(op.valid), torch.zeros_like(op.raw)
    ids, count, out = torch.zeros_like(op.ids), torch.zeros_like(op.count), torch.zeros_like(op.out)
    op.lib.call("prismkv_decode", q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(), op.bits.data_ptr(),
                k.data_ptr(), v.data_ptr(), work.data_ptr(), feats.data_ptr(), valid.data_ptr(), raw.data_ptr(),
                ids.data_ptr(), count.data_ptr(), out.data_ptr(), groups, op.history, k.shape[1] - op.history,
                op.capacity, op.row_words, k.stride(0), v.stride(0), op.capacity, nbytes(work),
                stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert int(work[:4].view(torch.int32)[0]) == 0  # no bounded wait gave up
    got = (feats.cpu().numpy(), valid.cpu().numpy(), raw.cpu().numpy(), ids.cpu().numpy(), count.cpu().numpy())
    for g in range(groups):
        assert np.array_equal(got[0][g], ref[0][g]) and np.array_equal(got[1][g], ref[1][g]), g
        assert got[2][g] == ref[2][g] and got[4][g] == ref[4][g], g
        assert np.array_equal(got[3][g][:got[4][g]], ref[3][g][:ref[4][g]]), g
    err = expect.attention_errors(bf16_bits(out)[:groups], want[:groups])
    log(f"  groups={groups}: {err}")
    assert err["rel_l2"] <= AV_TOL and err["max_abs"] < 0.05, err



@pytest.mark.parametrize("H", [4096, 65536, 200000])
def test_route_union_one_launch(H):
    # Native8B.route() runs prismkv_route_union (stages 1-2 in one launch):
    # features / valid / raw / ids / count bit-identical to the two-launch
    # route (prismkv_route_single, then prismkv_union_n), on repeated calls
    # and after a decode on the same workspace, which is left zero
    op, q, k, v = device_layer(H, 16, seed=12)
    lib, s = op.lib, torch.cuda.current_stream().cuda_stream

    def two():
        lib.call("prismkv_route_single", q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(),
                 op.decode_work.data_ptr(), op.features.data_ptr(), op.valid.data_ptr(), op.raw.data_ptr(), 8,
                 nbytes(op.decode_work), stream=s)
        lib.call("prismkv_union_n", op.bits.data_ptr(), op.features.data_ptr(), op.valid.data_ptr(),
                 op.union_work.data_ptr(), op.ids.data_ptr(), op.count.data_ptr(), 8, op.history, op.row_words,
                 op.capacity, 16, nbytes(op.union_work), stream=s)

    def outputs():
        torch.cuda.synchronize()
        f, va, r, ids, c = route_outputs(op)
        out = (f.copy(), va.copy(), r.copy(), [ids[g][:c[g]].copy() for g in range(8)], c.copy())
        for x in (op.features, op.valid, op.raw, op.ids, op.count):
            x.zero_()
        return out

    two()
    want = outputs()
    for step in range(3):
        op.route(q)
        got = outputs()
        for a, b in zip(want[:3], got[:3]):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), step
        assert np.array_equal(want[4], got[4]), step
        for g in range(8):
            assert np.array_equal(want[3][g], got[3][g]), (step, g)
        if step == 1:
            op(q, k, v)
            torch.cuda.synchronize()
    assert int(op.decode_work.view(torch.int32)[0]) == 0
    assert op.decode_errors() == 0
    assert not bool(op.decode_work[16:].any()), "the workspace is left zero"
    log(f"  H={H}: one-launch route equals route + union over 3 calls; unique ids {want[4].tolist()}")
