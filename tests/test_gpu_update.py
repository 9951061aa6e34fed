"""GPU parity of the incremental index update (append_index,
src/prismkv/core.py:186-201) against the CPU oracle.

For every group of each case:
  * activations relu((k - center)/scale W^T + b) match the oracle's
    double-accumulated encode within fp32 rounding;
  * the device's memberships equal the oracle's BatchTopK applied to the
    device's own activations -- bit-exact, including the flat-index tie rule
    (src/prismkv/core.py:13-26) -- and differ from the oracle's selection on
    its own activations only at values within the encode error of tau;
  * old memberships are untouched and new ones sit at columns H + t;
  * counts are old + new exactly; moments equal the oracle's Chan merge of the
    old moments with the block's population moments within fp32 rounding;
  * the decode path then runs on the updated tables and matches the oracle's
    route and attention over the exported index.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import bf16_to_f32, cases, expect
from tests.gpu_util import bf16_bits, bf16_tensor, device_indices, log, route_outputs
from tests.test_gpu_build import block_lists

pytestmark = pytest.mark.gpu

F = 3000


def run_append(case):
    from prismkv_amd import Native8B
    H, N, T = case["H"], case["N"], case["T"]
    op = Native8B(device_indices(case), capacity=H + N + T)
    op.set_encoder_tables(torch.from_numpy(case["W"]), torch.from_numpy(case["b"]), torch.from_numpy(case["scale"]),
                          case["key_mean"])
    k = bf16_tensor(case["k"])
    op.append(k, N)
    torch.cuda.synchronize()
    assert op.history == H + N
    return op, k


def lists_from_flat(flat, N, offset):
    sel = np.zeros(N * F, bool)
    sel[flat] = True
    sel = sel.reshape(N, F)
    return [np.flatnonzero(sel[:, f]) + offset for f in range(F)]


def check_group(case, g, act, got, tol_scale=1.0):
    H, N, km = case["H"], case["N"], case["key_mean"]
    old = case["indices"][g]
    kf = bf16_to_f32(case["k"][g])
    block = kf[H:H + N]
    ref_next, act_ref = oracle.build_index(block, case["W"][g], case["b"][g], float(case["scale"][g]), km,
                                           center=old.center, return_act=True)
    # activations
    err = float(np.abs(act - act_ref).max())
    bound = 2e-6 * max(1.0, float(np.abs(act_ref).max()))
    assert err <= bound, ("activation error", g, err, bound)
    # BatchTopK on the device's own activations: exact
    count = min(N * km, N * F)
    flat = oracle.positive_global_topk(act, count)
    new_lists = lists_from_flat(flat, N, H)
    for f in range(F):
        want = np.concatenate((old.lists[f], new_lists[f]))
        have = got.lists[f].numpy()
        if not np.array_equal(have, want):
            raise AssertionError(f"group {g} bucket {f}: lists differ ({len(have)} vs {len(want)})")
    # against the oracle's selection on its own activations: only values at tau may move
    ref_sel = np.zeros(N * F, bool)
    for f, l in enumerate(ref_next.lists):
        ref_sel[np.asarray(l) * F + f] = True
    dev_sel = np.zeros(N * F, bool)
    dev_sel[flat] = True
    moved = np.flatnonzero(ref_sel != dev_sel)
    if len(moved):
        vals = act_ref.reshape(-1)
        tau = np.partition(vals, vals.size - count)[vals.size - count]
        assert np.abs(vals[moved] - tau).max() <= 2 * err + 1e-7, ("selection moved away from tau", g)
    # counts exact, moments: Chan merge of old and the block's moments over the device's lists
    local = [l - H for l in new_lists]
    cb, mb, vb = oracle.summarize(block, local)
    co, mo, vo = oracle.merge_moments(old.counts, old.mean, old.variance, cb, mb, vb)
    assert np.array_equal(got.counts.cpu().numpy(), co), ("counts", g)
    scale = max(1.0, float(np.abs(kf).max()))
    m = got.mean.cpu().numpy()
    v = got.variance.cpu().numpy()
    assert np.allclose(m, mo, rtol=1e-4, atol=2e-5 * scale * tol_scale), ("mean", g, float(np.abs(m - mo).max()))
    assert np.allclose(v, vo, rtol=1e-4, atol=2e-5 * scale * scale * tol_scale), ("var", g, float(np.abs(v - vo).max()))
    return len(flat), len(moved), err


def check_decode_after(case, op, k, got):
    """Decode over the updated tables against the oracle on the exported index."""
    H2 = case["H"] + case["N"]
    idx = [oracle.Index(H2, i.center.cpu().numpy(), i.counts.cpu().numpy(), i.mean.cpu().numpy(),
                        i.variance.cpu().numpy(), [l.numpy() for l in i.lists]) for i in got]
    case2 = dict(H=H2, T=case["T"], q=case["q"], k=case["k"], v=case["v"], indices=idx, kind=case["kind"])
    q, v = bf16_tensor(case["q"]), bf16_tensor(case["v"])
    out = op(q, k, v)
    torch.cuda.synchronize()
    groups = expect.expected(case2)
    identical, near = expect.compare_route(groups, *route_outputs(op))
    assert identical + near == 8
    err = expect.attention_errors(bf16_bits(out), expect.expected_attention(case2, groups))
    log(f"  decode after append: {identical} identical, {near} near-tie; {err}")
    assert err["rel_l2"] <= 2e-3 and err["max_abs"] < 0.05, err


@pytest.mark.parametrize("kind", cases.UPDATE_KINDS)
def test_append_block(kind):
    case = cases.update_case(kind, H=512, N=256, T=8, seed=21)
    log(f"update case kind={kind} H={case['H']} N={case['N']}")
    op, k = run_append(case)
    act = op.update_activations(case["N"]).cpu().numpy()
    got = op.export_indices()
    for g in range(8):
        sel, moved, err = check_group(case, g, act[g], got[g])
        log(f"  group {g}: selected={sel} moved_at_tau={moved} act_err={err:.2e}")
        if kind == "bias_ties":
            # every value ties at 1: the budget is the first N*key_mean flat indices
            assert sel == case["N"] * case["key_mean"]
        if kind == "dead":
            assert sel == 0
    check_decode_after(case, op, k, got)


def test_append_full_block_4096():
    # the reference's update interval (src/prismkv/hf_reference.py:75,209-211)
    case = cases.update_case("random", H=1024, N=4096, T=16, seed=33)
    log(f"update case kind=random H={case['H']} N={case['N']}")
    op, k = run_append(case)
    act = op.update_activations(case["N"]).cpu().numpy()
    got = op.export_indices()
    for g in range(8):
        sel, moved, err = check_group(case, g, act[g], got[g])
        log(f"  group {g}: selected={sel} moved_at_tau={moved} act_err={err:.2e}")
    check_decode_after(case, op, k, got)


@pytest.mark.parametrize("N", [1, 37, 100])
def test_append_ragged_block(N):
    # a block that fills neither a 16-row wave tile nor a 128-token encode
    # workgroup: the rows past the block are masked at the activation store
    case = cases.update_case("random", H=700, N=N, T=3, seed=50 + N)
    log(f"update case kind=random H={case['H']} N={case['N']}")
    op, k = run_append(case)
    act = op.update_activations(case["N"]).cpu().numpy()
    got = op.export_indices()
    for g in range(8):
        sel, moved, err = check_group(case, g, act[g], got[g])
        log(f"  group {g}: selected={sel} moved_at_tau={moved} act_err={err:.2e}")
    check_decode_after(case, op, k, got)


def test_catch_up_two_blocks():
    # two consecutive appends equal two oracle append_index steps
    H, N, T = 300, 128, 5
    case = cases.update_case("random", H=H, N=2 * N, T=T, seed=41)
    from prismkv_amd import Native8B
    op = Native8B(device_indices(case), capacity=H + 2 * N + T)
    op.set_encoder_tables(torch.from_numpy(case["W"]), torch.from_numpy(case["b"]), torch.from_numpy(case["scale"]),
                          case["key_mean"])
    k = bf16_tensor(case["k"])
    assert op.catch_up(k, total=H + 2 * N + T, update_interval=N) == 2
    assert op.history == H + 2 * N
    torch.cuda.synchronize()
    got = op.export_indices()
    kf = bf16_to_f32(case["k"])
    for g in range(8):
        idx = case["indices"][g]
        W, b, s = case["W"][g], case["b"][g], float(case["scale"][g])
        have = [l.numpy() for l in got[g].lists]
        moved = 0
        for blk in range(2):
            lo = idx.history
            xb = (kf[g, lo:lo + N] - idx.center) / np.float32(s)
            idx, act = oracle.append_index(idx, kf[g, lo:lo + N], W, b, s, case["key_mean"], return_act=True)
            # each block's memberships are its own BatchTopK: any difference lies within rounding of its tau
            moved += expect.check_memberships(block_lists(idx.lists, lo, N), block_lists(have, lo, N), act,
                                              N * case["key_mean"], expect.encode_error_bound(xb, W, b),
                                              f"group {g} block {blk}")
        same = all(np.array_equal(x, y) for x, y in zip(have, idx.lists))
        log(f"  group {g}: lists identical={same}, memberships differing (within rounding of tau): {moved}")
        if same:
            assert np.array_equal(got[g].counts.cpu().numpy(), idx.counts)
            assert np.allclose(got[g].mean.cpu().numpy(), idx.mean, rtol=1e-4, atol=1e-4)
            assert np.allclose(got[g].variance.cpu().numpy(), idx.variance, rtol=1e-4, atol=1e-4)


def test_append_smaller_block_after_larger():
    # one workspace serves blocks of different sizes (the zeroed histograms
    # and control words sit at offsets that do not move with the block size):
    # a 256-key block, then a 37-key block, each against the oracle
    from prismkv_amd import Native8B
    H, N1, N2, T = 700, 256, 37, 3
    case = cases.update_case("random", H=H, N=N1 + N2, T=T, seed=57)
    op = Native8B(device_indices(case), capacity=H + N1 + N2 + T)
    op.set_encoder_tables(torch.from_numpy(case["W"]), torch.from_numpy(case["b"]), torch.from_numpy(case["scale"]),
                          case["key_mean"])
    k = bf16_tensor(case["k"])
    op.append(k, N1)
    torch.cuda.synchronize()
    mid = [oracle.Index(H + N1, i.center.cpu().numpy(), i.counts.cpu().numpy(), i.mean.cpu().numpy(),
                        i.variance.cpu().numpy(), [l.numpy() for l in i.lists]) for i in op.export_indices()]
    op.append(k, N2)
    torch.cuda.synchronize()
    assert op.history == H + N1 + N2
    act = op.update_activations(N2).cpu().numpy()
    got = op.export_indices()
    case2 = dict(case, H=H + N1, N=N2, indices=mid)
    for g in range(8):
        sel, moved, err = check_group(case2, g, act[g], got[g])
        log(f"  group {g}: second block selected={sel} moved_at_tau={moved} act_err={err:.2e}")
        assert sel == N2 * case["key_mean"]
