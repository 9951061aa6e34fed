"""Bounded inter-workgroup waits on the product path.

Every wait of the decode and union kernels gives up after a host-settable
number of sleeps and marks an error word instead of hanging.  These tests
force a give-up from the host (spin limit 0: a wait gives up at its first
check if the words it needs have not landed), with every kernel still
running to its end, and check that the binding raises RuntimeError, resets
its workspaces, and decodes correctly again once the limit is restored.
"""
import pytest
import torch

from oracle import cases, expect
from prismkv_amd import set_spin_limit
from tests.gpu_util import bf16_bits, log, operator, route_outputs

pytestmark = pytest.mark.gpu

DEFAULT_LIMIT = 1 << 20


def _forced_give_up(call, op, attempts=3):
    """Runs `call` under spin limit 0 until the binding reports a give-up;
    returns the attempt at which it raised (None if it never did)."""
    previous = set_spin_limit(0)
    assert previous == DEFAULT_LIMIT
    try:
        for attempt in range(attempts):
            call()
            torch.cuda.synchronize()
            try:
                op.check_errors()
            except RuntimeError as exc:
                log(f"  attempt {attempt}: {exc}")
                return attempt
    finally:
        set_spin_limit(previous)
    return None


def _check_decode(op, q, k, v, case):
    out = op(q, k, v)
    torch.cuda.synchronize()
    groups = expect.expected(case)
    identical, near = expect.compare_route(groups, *route_outputs(op))
    err = expect.attention_errors(bf16_bits(out), expect.expected_attention(case, groups))
    log(f"  after reset: identical={identical} near={near} {err}")
    assert identical == 8 and near == 0
    assert err["rel_l2"] <= 2e-3
    assert op.decode_errors() == 0


def test_decode_give_up_raises_and_recovers():
    case = cases.native_case(4096, 64, "random")
    op, q, k, v = operator(case)
    op(q, k, v)
    torch.cuda.synchronize()
    assert op.decode_errors() == 0
    attempt = _forced_give_up(lambda: op(q, k, v), op)
    assert attempt is not None, "no wait gave up under spin limit 0"
    # the binding reset everything: the error words are clear and the next call is exact
    assert op.decode_errors() == 0
    _check_decode(op, q, k, v, case)


def test_route_give_up_raises_on_next_call():
    """A give-up noticed by the NEXT call's entry check (no explicit check)."""
    case = cases.native_case(4096, 64, "random")
    op, q, k, v = operator(case)
    previous = set_spin_limit(0)
    try:
        raised = False
        for _ in range(4):
            try:
                op.route(q)
                torch.cuda.synchronize()
            except RuntimeError as exc:
                log(f"  route raised: {exc}")
                raised = True
                break
    finally:
        set_spin_limit(previous)
    assert raised
    _check_decode(op, q, k, v, case)


def test_attention_give_up_raises_and_recovers():
    """The separate attention (prismkv_attend on the decode's attention
    phases) reports a give-up through its workspace's error word."""
    case = cases.native_case(4096, 64, "random")
    op, q, k, v = operator(case)
    op.route(q)
    op.attention(q, k, v)
    torch.cuda.synchronize()
    assert op.decode_errors() == 0
    attempt = _forced_give_up(lambda: op.attention(q, k, v), op)
    assert attempt is not None, "no wait gave up under spin limit 0"
    assert op.decode_errors() == 0
    op.route(q)
    out = op.attention(q, k, v)
    torch.cuda.synchronize()
    groups = expect.expected(case)
    err = expect.attention_errors(bf16_bits(out), expect.expected_attention(case, groups))
    log(f"  attention after reset: {err}")
    assert err["rel_l2"] <= 2e-3
    assert op.decode_errors() == 0


def test_core_attend_give_up_raises():
    """core.attend checks the error word after its launch and raises."""
    from prismkv_amd import core
    case = cases.native_case(2048, 16, "random")
    op, q, k, v = operator(case)
    ids = torch.arange(0, 2048, 3, device="cuda")
    previous = set_spin_limit(0)
    try:
        raised = False
        for _ in range(4):
            try:
                core.attend(q[0], k[0], v[0], ids, 2048)
            except RuntimeError as exc:
                log(f"  core.attend raised: {exc}")
                raised = True
                break
    finally:
        set_spin_limit(previous)
    assert raised
    out = core.attend(q[0], k[0], v[0], ids, 2048)
    assert torch.isfinite(out.float()).all()


def test_undersized_workspace_is_refused_before_any_launch():
    # a workspace one byte short of prismkv_decode_work_bytes (e.g. one sized
    # under an older layout) is refused with -1 by every decode variant and
    # nothing is enqueued: the outputs keep the sentinel written before
    from prismkv_amd._lib import nbytes
    case = cases.native_case(2048, 16, "random", seed=17)
    op, q, k, v = operator(case)
    out = op(q, k, v).clone()
    torch.cuda.synchronize()
    short = nbytes(op.decode_work) - 1
    s = torch.cuda.current_stream().cuda_stream
    tail = torch.tensor([16], dtype=torch.int32, device="cuda")
    T = k.shape[1] - op.history
    common = (op.row_words, k.stride(0), v.stride(0), op.capacity, short)
    head = (q.data_ptr(), op.moments.data_ptr(), op.n.data_ptr(), op.bits.data_ptr(), k.data_ptr(), v.data_ptr(),
            op.decode_work.data_ptr(), op.features.data_ptr(), op.valid.data_ptr(), op.raw.data_ptr(),
            op.ids.data_ptr(), op.count.data_ptr(), op.out.data_ptr())
    given = (q.data_ptr(), op.bits.data_ptr(), k.data_ptr(), v.data_ptr(), op.decode_work.data_ptr(),
             op.features.data_ptr(), op.valid.data_ptr(), op.ids.data_ptr(), op.count.data_ptr(), op.out.data_ptr())
    calls = {
        "prismkv_decode": (*head, 8, op.history, T, op.capacity, *common),
        "prismkv_decode_tail": (*head, tail.data_ptr(), 8, op.history, T, op.capacity, *common),
        "prismkv_decode_capped": (*head, 8, op.history, T, op.capacity, 100, *common),
        "prismkv_decode_capped_tail": (*head, tail.data_ptr(), 8, op.history, T, op.capacity, 100, *common),
        "prismkv_union_attend": (*given, 8, op.history, T, op.capacity, *common),
        "prismkv_union_attend_tail": (*given, tail.data_ptr(), 8, op.history, T, op.capacity, *common),
        "prismkv_route_single": (*head[:3], op.decode_work.data_ptr(), op.features.data_ptr(), op.valid.data_ptr(),
                                 op.raw.data_ptr(), 8, short),
    }
    for name, args in calls.items():
        op.out.fill_(7.0)
        op.count.fill_(-5)
        op.features.fill_(-3)
        torch.cuda.synchronize()
        assert getattr(op.lib.cdll, name)(*args, s) == -1, name
        torch.cuda.synchronize()
        assert bool((op.out == 7.0).all()) and bool((op.count == -5).all()) and bool((op.features == -3).all()), name
    log(f"  refused without a launch: {sorted(calls)}")
    assert torch.equal(op(q, k, v), out)
    assert op.decode_errors() == 0


def test_attention_reports_ids_out_of_range():
    # Native8B.attention reads `ids` / `count` as route() left them; an id
    # outside [0, history) (or a count outside [0, history]) is read clamped,
    # so every access stays in range, and the error word makes the next check
    # raise instead of returning a plausible but wrong output
    case = cases.native_case(4096, 40, "random", seed=23)
    op, q, k, v = operator(case)
    op.route(q)
    good = op.attention(q, k, v).clone()
    torch.cuda.synchronize()
    assert op.decode_errors() == 0
    for what in ("id", "count"):
        op.route(q)
        if what == "id":
            op.ids[3, 0] = op.history + 5
        else:
            op.count[5] = op.history + 1
        op.attention(q, k, v)
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError, match="outside"):
            op.check_errors()
        log(f"  {what} out of range: reported")
    op.route(q)
    assert torch.equal(op.attention(q, k, v), good)
    assert op.decode_errors() == 0
