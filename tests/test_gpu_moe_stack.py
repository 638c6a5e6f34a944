"""The persistent decode (hk_moe_decode_stack as one cooperative launch with
flag-tagged hand-offs, stack_launch = HK_STACK_PERSISTENT) against the
per-layer launches: the same bits, layer ids and weights, over repeated calls
(the tags advance), and the same status bits for a non-finite hidden state.
Both paths are checked against the oracle at config 4's full 48 layers in
test_gpu_c4_stack.py."""
import sys

import numpy as np
import pytest

from tests import hk_testutil as U

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    from hawking_amd.runtime import Context
    return Context(0)


SHAPES = [
    # (label, n_layers, hidden, inter, shared_inter, experts, top_k, kind, group, shared_gate)
    ("config4-geometry", 4, 2048, 512, 512, 512, 10, U.HK_MIXED, 128, True),
    ("config3-geometry", 3, 2048, 512, 512, 512, 10, U.HK_Q4, 32, True),
    ("small-mixed-no-shared", 3, 512, 384, 0, 32, 5, U.HK_MIXED, 128, False),
    ("small-q4-wide-ungated-shared", 3, 512, 128, 256, 64, 6, U.HK_Q4, 64, False),
]


def run_mode(m, hd, persistent):
    """One token with the persistent launch (HK_STACK_PERSISTENT) or the
    per-layer launches (HK_STACK_PER_LAYER, the default)."""
    m.set_stack_launch(1 if persistent else 0)
    try:
        return m.forward_token(hd)
    finally:
        m.set_stack_launch(0)


def admitted(m):
    m.set_stack_launch(1)
    try:
        return m.stack_is_persistent()
    finally:
        m.set_stack_launch(0)


@pytest.mark.parametrize("label,n,H,I,SI,E,K,kind,group,gate", SHAPES)
def test_persistent_stack_bit_exact_vs_per_layer(ctx, label, n, H, I, SI, E, K, kind, group, gate):
    from hawking_amd.moe import MoeModel, MoeShape
    say("persistent stack", label)
    shape = MoeShape(n_layers=n, hidden=H, inter=I, shared_inter=SI, n_experts=E, top_k=K, expert_kind=kind,
                     expert_group=group, shared_gate=gate)
    m = MoeModel(ctx, shape)
    m.fill_synthetic(U.SEED + n)
    assert admitted(m), "the persistent launch must be admitted for this shape"
    ctx.device_status()  # clear
    rng = np.random.default_rng(7)
    for call in range(3):  # the tags advance from call to call
        h = rng.standard_normal(H).astype(np.float32) * (1.0 + call)
        out, ids, w = run_mode(m, h, True)
        rout, rids, rw = run_mode(m, h, False)
        assert np.array_equal(ids, rids), (label, call)
        assert np.array_equal(w.view(np.uint32), rw.view(np.uint32)), (label, call)
        assert np.array_equal(out.view(np.uint32), rout.view(np.uint32)), (label, call)
    assert ctx.device_status() == 0


def test_persistent_stack_flags_nonfinite_then_recovers(ctx):
    from hawking_amd.moe import MoeModel, MoeShape
    say("persistent stack non-finite")
    shape = MoeShape(n_layers=2, hidden=512, inter=128, shared_inter=128, n_experts=16, top_k=4,
                     expert_kind=U.HK_Q4, expert_group=32)
    m = MoeModel(ctx, shape)
    m.fill_synthetic(U.SEED)
    assert admitted(m)
    ctx.device_status()
    h = np.ones(512, np.float32)
    h[3] = np.nan
    run_mode(m, h, True)
    assert ctx.device_status() & 1
    h = np.random.default_rng(3).standard_normal(512).astype(np.float32)
    out, ids, w = run_mode(m, h, True)
    rout, rids, rw = run_mode(m, h, False)
    assert ctx.device_status() == 0
    assert np.array_equal(out.view(np.uint32), rout.view(np.uint32))


def test_persistent_stack_gives_up_and_recovers(ctx):
    """The persistent launch's give-up path, forced from the host: with a
    stall bound of 0 polls, the first wait that finds its producer's words
    missing gives up (status bit 4) and every other wait of the launch
    returns, so the launch drains (the call returns and the device answers);
    the next call, with a new tag and the default bound, is bit-identical to
    the per-layer launches."""
    from hawking_amd.moe import MoeModel, MoeShape
    say("persistent stack forced give-up")
    shape = MoeShape(n_layers=4, hidden=2048, inter=512, shared_inter=512, n_experts=512, top_k=10,
                     expert_kind=U.HK_MIXED, expert_group=128)
    m = MoeModel(ctx, shape)
    m.fill_synthetic(U.SEED + 4)
    assert admitted(m)
    h = np.random.default_rng(21).standard_normal(shape.hidden).astype(np.float32)
    ctx.device_status()
    m.set_stall_polls(0)
    try:
        run_mode(m, h, True)
    finally:
        m.set_stall_polls(65536)
    assert ctx.device_status() & 4, "a wait gave up: status bit 4"
    out, ids, w = run_mode(m, h, True)
    assert ctx.device_status() == 0
    rout, rids, rw = run_mode(m, h, False)
    assert np.array_equal(ids, rids)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    assert np.array_equal(out.view(np.uint32), rout.view(np.uint32))
