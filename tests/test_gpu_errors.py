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
