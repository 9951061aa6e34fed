"""GPU parity of the prefill index build (build_index,
src/prismkv/core.py:92-103) against the CPU oracle.

For every group of each case:
  * the device center equals the exact mean of the K rows rounded to fp32
    (to one ulp);
  * activations relu((k - center)/scale W^T + b) match the oracle's
    double-accumulated encode (with the device center) within fp32 rounding;
  * the device's memberships equal the oracle's BatchTopK applied to the
    device's own activations -- bit-exact, including the flat-index tie rule
    (src/prismkv/core.py:13-26) -- and differ from the oracle's selection on
    its own activations only at values within the encode error of tau;
  * counts equal the list lengths and the moments equal the oracle's
    summarize (src/prismkv/core.py:76-89) over the device's lists;
  * the decode path on the built tables matches the oracle's route and
    attention over the exported index.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import bf16_to_f32, cases, expect
from tests.gpu_util import bf16_bits, bf16_tensor, log, route_outputs

pytestmark = pytest.mark.gpu

F = 3000


def run_build(case, **kwargs):
    from prismkv_amd import Native8B
    k = bf16_tensor(case["k"])
    kwargs.setdefault("keep_activations", True)
    op = Native8B.from_keys(k, case["H"], torch.from_numpy(case["W"]), torch.from_numpy(case["b"]),
                            torch.from_numpy(case["scale"]), case["key_mean"], capacity=case["H"] + case["T"],
                            **kwargs)
    torch.cuda.synchronize()
    return op, k


def lists_from_flat(flat, H):
    tok, feat = flat // F, flat % F
    order = np.lexsort((tok, feat))
    return np.split(tok[order], np.cumsum(np.bincount(feat, minlength=F))[:-1])


def check_center(case, g, center):
    kf = bf16_to_f32(case["k"][g, :case["H"]])
    exact = kf.astype(np.float64).mean(0)
    err = np.abs(center.astype(np.float64) - exact)
    assert (err <= np.spacing(np.abs(exact).astype(np.float32)) + 1e-30).all(), ("center", g, float(err.max()))


def block_lists(lists, lo, n):
    """Per-feature lists restricted to tokens [lo, lo + n), shifted to start at 0."""
    out = []
    for l in lists:
        l = np.asarray(l, np.int64)
        out.append(l[(l >= lo) & (l < lo + n)] - lo)
    return out


def check_selection(case, g, act, got, ref=None):
    """Exact BatchTopK on the device activations; returns (selected, moved)."""
    H, km = case["H"], case["key_mean"]
    count = min(H * km, H * F)
    flat = oracle.positive_global_topk(act, count)
    want = lists_from_flat(flat, H)
    for f in range(F):
        have = got.lists[f].numpy()
        if not np.array_equal(have, want[f]):
            raise AssertionError(f"group {g} bucket {f}: lists differ ({len(have)} vs {len(want[f])})")
    moved = 0
    if ref is not None:
        ref_index, act_ref, err = ref
        ref_sel = np.zeros(H * F, bool)
        for f, l in enumerate(ref_index.lists):
            ref_sel[np.asarray(l) * F + f] = True
        dev_sel = np.zeros(H * F, bool)
        dev_sel[flat] = True
        idx = np.flatnonzero(ref_sel != dev_sel)
        moved = len(idx)
        if moved:
            vals = act_ref.reshape(-1)
            tau = np.partition(vals, vals.size - count)[vals.size - count]
            assert np.abs(vals[idx] - tau).max() <= 2 * err + 1e-7, ("selection moved away from tau", g)
    return len(flat), moved


def check_moments(case, g, got):
    kf = bf16_to_f32(case["k"][g, :case["H"]])
    lists = [l.numpy() for l in got.lists]
    c, m, v = oracle.summarize(kf, lists)
    assert np.array_equal(got.counts.cpu().numpy(), c), ("counts", g)
    s = max(1.0, float(np.abs(kf).max()))
    gm, gv = got.mean.cpu().numpy(), got.variance.cpu().numpy()
    assert np.allclose(gm, m, rtol=1e-6, atol=1e-7 * s), ("mean", g, float(np.abs(gm - m).max()))
    assert np.allclose(gv, v, rtol=1e-6, atol=1e-7 * s * s), ("var", g, float(np.abs(gv - v).max()))


def check_decode(case, op, k, got):
    H = case["H"]
    idx = [oracle.Index(H, i.center.cpu().numpy(), i.counts.cpu().numpy(), i.mean.cpu().numpy(),
                        i.variance.cpu().numpy(), [l.numpy() for l in i.lists]) for i in got]
    case2 = dict(H=H, T=case["T"], q=case["q"], k=case["k"], v=case["v"], indices=idx, kind=case["kind"])
    q, v = bf16_tensor(case["q"]), bf16_tensor(case["v"])
    out = op(q, k, v)
    torch.cuda.synchronize()
    assert op.decode_errors() == 0
    groups = expect.expected(case2)
    identical, near = expect.compare_route(groups, *route_outputs(op))
    assert identical + near == 8
    err = expect.attention_errors(bf16_bits(out), expect.expected_attention(case2, groups))
    log(f"  decode on the built index: {identical} identical, {near} near-tie; {err}")
    assert err["rel_l2"] <= 2e-3 and err["max_abs"] < 0.05, err


def full_check(case, op, k, center_given=False):
    H, km = case["H"], case["key_mean"]
    act = op.build_activations().cpu().numpy()
    centers = op.center.cpu().numpy()
    got = op.export_indices()
    for g in range(8):
        if not center_given:
            check_center(case, g, centers[g])
        kf = bf16_to_f32(case["k"][g, :H])
        ref_index, act_ref = oracle.build_index(kf, case["W"][g], case["b"][g], float(case["scale"][g]), km,
                                                center=centers[g], return_act=True)
        err = float(np.abs(act[g] - act_ref).max())
        bound = 2e-6 * max(1.0, float(np.abs(act_ref).max()))
        assert err <= bound, ("activation error", g, err, bound)
        sel, moved = check_selection(case, g, act[g], got[g], (ref_index, act_ref, err))
        check_moments(case, g, got[g])
        log(f"  group {g}: selected={sel} moved_at_tau={moved} act_err={err:.2e}")
        if case["kind"] == "bias_ties":
            assert sel == min(H * km, H * F)
        if case["kind"] == "dead":
            assert sel == 0
    return got


@pytest.mark.parametrize("kind", cases.UPDATE_KINDS)
def test_build_kinds(kind):
    case = cases.build_case(kind, H=600, T=5, seed=61)
    log(f"build case kind={kind} H={case['H']}")
    op, k = run_build(case)
    got = full_check(case, op, k)
    if kind != "dead":
        check_decode(case, op, k, got)


@pytest.mark.parametrize("H", [1, 33, 2048])
def test_build_sizes(H):
    # one key (budget 8 of 3000 values; a computed center would equal the key
    # and zero every activation, so it gets a zero center), a partial bitmap
    # word, and a 4-chunk row
    case = cases.build_case("random", H=H, T=3, seed=70 + H)
    log(f"build case kind=random H={H}")
    center = torch.zeros(8, 128, device="cuda") if H == 1 else None
    op, k = run_build(case, center=center)
    got = full_check(case, op, k, center_given=center is not None)
    assert all(x.memberships == 8 * H for x in got)


def test_build_given_center_and_batches():
    # center supplied by the caller (flags 0), and groups indexed one batch at a
    # time: the tables equal those of an all-groups batch bit for bit
    case = cases.build_case("random", H=700, T=4, seed=81)
    center = torch.from_numpy(np.linspace(-0.1, 0.1, 8 * 128, dtype=np.float32).reshape(8, 128)).cuda()
    op1, k = run_build(case, center=center, keep_activations=False)
    assert op1.build_batch == 8
    assert torch.equal(op1.center, center)
    per_group = op1.lib.query("prismkv_build_work_bytes", 1, case["H"])
    op2, _ = run_build(case, center=center, work_limit=3 * per_group, keep_activations=False)
    assert op2.build_batch == 3
    torch.cuda.synchronize()
    for name in ("bits", "n", "moments", "center"):
        assert torch.equal(getattr(op1, name), getattr(op2, name)), name
    # against the oracle with the same center
    got = op1.export_indices()
    for g in (0, 5):
        kf = bf16_to_f32(case["k"][g, :case["H"]])
        ref = oracle.build_index(kf, case["W"][g], case["b"][g], float(case["scale"][g]), case["key_mean"],
                                 center=center[g].cpu().numpy())
        x = (kf - center[g].cpu().numpy()) / np.float32(case["scale"][g])
        act = oracle.sae_dense(x, case["W"][g], case["b"][g])
        moved = expect.check_memberships(ref.lists, [l.numpy() for l in got[g].lists], act,
                                         case["H"] * case["key_mean"],
                                         expect.encode_error_bound(x, case["W"][g], case["b"][g]), f"group {g}")
        log(f"  group {g}: memberships differing from the oracle build (all within rounding of tau): {moved}")
        check_moments(case, g, got[g])


def test_build_then_append():
    # build_index over H keys, then append_index of one block: the oracle's two steps
    from prismkv_amd.native8b import MAX_BLOCK
    H, N, T = 900, 256, 6
    case = cases.build_case("random", H=H + N, T=T, seed=91)
    case_b = dict(case, H=H, T=N + T)
    op, k = run_build(case_b, keep_activations=False)
    op.append(k, N)
    torch.cuda.synchronize()
    assert op.history == H + N and N <= MAX_BLOCK
    got = op.export_indices()
    kf = bf16_to_f32(case["k"])
    for g in range(8):
        W, b, s = case["W"][g], case["b"][g], float(case["scale"][g])
        idx0 = oracle.build_index(kf[g, :H], W, b, s, case["key_mean"], center=op.center[g].cpu().numpy())
        idx1, act = oracle.append_index(idx0, kf[g, H:H + N], W, b, s, case["key_mean"], return_act=True)
        same = all(np.array_equal(a.numpy(), b_) for a, b_ in zip(got[g].lists, idx1.lists))
        x = (kf[g, H:H + N] - op.center[g].cpu().numpy()) / np.float32(s)
        moved = expect.check_memberships(block_lists(idx1.lists, H, N), block_lists(got[g].lists, H, N), act,
                                         N * case["key_mean"], expect.encode_error_bound(x, W, b), f"group {g}")
        log(f"  group {g}: lists identical={same}, block memberships differing (within rounding of tau): {moved}")
        if same:
            assert np.array_equal(got[g].counts.cpu().numpy(), idx1.counts)
            assert np.allclose(got[g].mean.cpu().numpy(), idx1.mean, rtol=1e-4, atol=1e-5)
            assert np.allclose(got[g].variance.cpu().numpy(), idx1.variance, rtol=1e-4, atol=1e-5)


def test_build_64k():
    # the 8B geometry's history: 65536 keys per group, 8 groups in one batch
    # (6.3 GB of activations); activations checked on a row sample, selection
    # exact on the device activations of three groups, moments of all groups
    H = 65536
    case = cases.build_case("random", H=H, T=32, seed=101)
    log(f"build case kind=random H={H}")
    op, k = run_build(case)
    assert op.build_batch == 8
    centers = op.center.cpu().numpy()
    got = op.export_indices()
    rows = np.random.default_rng(5).choice(H, 256, replace=False)
    for g in range(8):
        check_center(case, g, centers[g])
        kf = bf16_to_f32(case["k"][g, :H])
        x = (kf[rows] - centers[g]) / case["scale"][g]
        act_rows = op.build_activations()[g, torch.from_numpy(rows).cuda()].cpu().numpy()
        ref_rows = oracle.sae_dense(x, case["W"][g], case["b"][g])
        err = float(np.abs(act_rows - ref_rows).max())
        assert err <= 2e-6 * max(1.0, float(np.abs(ref_rows).max())), ("activation error", g, err)
        if g in (0, 3, 7):
            sel, _ = check_selection(case, g, op.build_activations()[g].cpu().numpy(), got[g])
            assert sel == H * case["key_mean"]
        check_moments(case, g, got[g])
        log(f"  group {g}: memberships={got[g].memberships} act_err={err:.2e}")
    check_decode(case, op, k, got)


def test_build_ties_over_many_ranges():
    # W = 0, b = 1 on buckets 0..8 only: every key has exactly 9 positive
    # activations, all equal to 1, against a budget of 8 per key, so tau = 1
    # and the ties overflow.  The first 8 H ties in flat order (token * 3000 +
    # bucket, core.py:23-24) are all 9 buckets of tokens t < 8H // 9 and the
    # first 8H mod 9 buckets of token 8H // 9.  At H = 8192 the ties span 333
    # of the 375 contiguous ranges the tie kernels cut the activations into,
    # more than one workgroup per range.
    H = 8192
    case = cases.build_case("bias_ties", H=H, T=2, seed=111)
    case["b"][:] = 0.0
    case["b"][:, :9] = 1.0
    op, k = run_build(case, keep_activations=False)
    got = op.export_indices()
    full, part = divmod(8 * H, 9)
    for g in range(8):
        for f in range(3000):
            want = np.arange(full + (1 if f < part else 0)) if f < 9 else np.zeros(0, np.int64)
            assert np.array_equal(got[g].lists[f].numpy(), want), (g, f)
        check_moments(case, g, got[g])
    log(f"  ties over many ranges: {got[0].memberships} memberships per group")


def test_long_history_with_updates():
    # H = 131072 built on the device (two group batches within the 8 GiB
    # workspace), then the tail grows 0 -> 4096 with an update every 1024
    # tokens (src/prismkv/hf_reference.py:209-211 with interval 1024): decode
    # at several tail lengths against the oracle on the exported index
    H, T = 131072, 4096
    case = cases.build_case("random", H=H, T=T, seed=131)
    op, k = run_build(dict(case, T=T), keep_activations=False)
    assert op.build_batch == 5
    v, q = bf16_tensor(case["v"]), bf16_tensor(case["q"])
    for tail in (0, 1, 1025, 3000, 4096):
        total = H + tail
        op.catch_up(k[:, :total], total, update_interval=1024)
        want = H + max(0, (tail - 1) // 1024) * 1024
        assert op.history == want, (tail, op.history, want)
        out = op(q, k[:, :total], v[:, :total])
        torch.cuda.synchronize()
        assert op.decode_errors() == 0
        got = op.export_indices()
        idx = [oracle.Index(op.history, i.center.cpu().numpy(), i.counts.cpu().numpy(), i.mean.cpu().numpy(),
                            i.variance.cpu().numpy(), [l.numpy() for l in i.lists]) for i in got]
        c2 = dict(H=op.history, T=total - op.history, q=case["q"], k=case["k"][:, :total],
                  v=case["v"][:, :total], indices=idx, kind="random")
        groups = expect.expected(c2)
        identical, near = expect.compare_route(groups, *route_outputs(op))
        assert identical + near == 8
        err = expect.attention_errors(bf16_bits(out), expect.expected_attention(c2, groups))
        log(f"  tail {tail}: history={op.history} {identical} identical, {near} near-tie; {err}")
        assert err["rel_l2"] <= 2e-3 and err["max_abs"] < 0.05, err


def test_stress_mixture_keys_with_cap():
    # the stress configuration: H = 262144 keys per group drawn from a
    # 64-component Gaussian mixture (centers ~ N(0, I), sigma = 0.3), indexed
    # on the device (4 batches of 2 groups within the 8 GiB workspace), then
    # routed with the strict unique-ID cap floor(H / 16) = 16384
    # (src/prismkv/core.py:149-163): the device's ranked order is checked
    # against the oracle, then fed to the oracle's budgeted walk, which the
    # device's kept buckets / raw / ids must equal bit for bit
    H, T, cap = 262144, 16, 1 / 16
    gen = torch.Generator(device="cuda").manual_seed(151)
    centers = torch.randn(8, 64, 128, generator=gen, device="cuda")
    comp = torch.randint(0, 64, (8, H + T), generator=gen, device="cuda")
    noise = torch.randn(8, H + T, 128, generator=gen, device="cuda") * 0.3
    k = (torch.gather(centers, 1, comp[..., None].expand(-1, -1, 128)) + noise).to(torch.bfloat16)
    v = torch.randn(8, H + T, 128, generator=gen, device="cuda").to(torch.bfloat16)
    q = torch.randn(8, 4, 128, generator=gen, device="cuda").to(torch.bfloat16)
    del noise
    base = cases.build_case("random", H=1, T=0, seed=152)  # per-group SAE tables and scales
    from prismkv_amd import Native8B
    op = Native8B.from_keys(k, H, torch.from_numpy(base["W"]), torch.from_numpy(base["b"]),
                            torch.from_numpy(base["scale"]), 8, capacity=H + T)
    torch.cuda.synchronize()
    assert op.build_batch == 2
    got = op.export_indices()
    idx = [oracle.Index(H, i.center.cpu().numpy(), i.counts.cpu().numpy(), i.mean.cpu().numpy(),
                        i.variance.cpu().numpy(), [l.numpy() for l in i.lists]) for i in got]
    case = dict(H=H, T=T, q=bf16_bits(q), k=bf16_bits(k), v=bf16_bits(v), indices=idx, kind="mixture")
    op.route(q)
    identical, near = expect.compare_route(expect.expected(case), *route_outputs(op))
    assert identical + near == 8
    features, valid, _, _, _ = route_outputs(op)
    orders = [features[g][valid[g] > 0] for g in range(8)]
    op.unique_cap = cap
    out = op(q, k, v)
    torch.cuda.synchronize()
    f2, v2, r2, i2, c2 = route_outputs(op)
    want, skipped = [], 0
    for g in range(8):
        ids, meta = oracle.select_buckets(orders[g], idx[g].lists, H, cap)
        nf = len(meta["features"])
        skipped += len(orders[g]) - nf
        assert meta["limit"] == 16384
        assert f2[g][:nf].tolist() == meta["features"], ("kept buckets", g)
        assert int(r2[g]) == meta["raw"] and int(c2[g]) == len(ids), ("raw/count", g)
        assert np.array_equal(i2[g][:len(ids)].astype(np.int64), ids), ("ids", g)
        want.append(dict(ids=ids))
    sizes = [max(len(l) for l in i.lists) for i in idx]
    log(f"  largest bucket per group {sizes}; {skipped} ranked buckets skipped by the cap; unique {c2.tolist()}")
    err = expect.attention_errors(bf16_bits(out), expect.expected_attention(case, want))
    log(f"  capped decode {err}")
    assert err["rel_l2"] <= 2e-3 and err["max_abs"] < 0.05, err
