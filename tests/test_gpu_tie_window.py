"""The router tie window (route_tie_epsilon, crates/hawking-core/src/moe.rs:8-14,
applied by source_qwen80_topk_router, model/qwen80_complete_runtime.rs:5988-6000)
inside the fused decode kernels: hk_moe_decode_layer (the in-block wave top-k of
the gate/up kernel), the persistent hk_moe_decode_stack (its route and down
roles rank too) and hk_moe15_decode_layer, each against the oracle's serial
scan with the same window.

The window is chosen per input so that it changes the selection (the strict
rule would pick other ids, or the same ids in another order) and so that every
pairwise difference of the normalised probabilities stays away from it
(tie_window_margin_ok); otherwise the input advances."""
import sys

import numpy as np
import pytest

from tests import hk_testutil as U

pytestmark = pytest.mark.gpu
TOL = 2e-5


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    from hawking_amd.runtime import Context
    return Context(0)


def discriminating_window(oracle, logits, k):
    """A tie window that changes the top-k of these logits and keeps the margin
    rule, or None."""
    l64 = logits.astype(np.float64)
    q = np.exp(l64 - l64.max())
    q /= q.sum()
    top = np.sort(q)[::-1][:k + 4]
    gaps = top[:-1] - top[1:]
    strict, _ = oracle.router_softmax_topk(logits, k, 0.0)
    for f in (1.5, 2.5, 4.0, 6.0, 9.0):
        eps = float(np.median(gaps) * f)
        tie, _ = oracle.router_softmax_topk(logits, k, eps)
        if tie.tolist() != strict.tolist() and U.tie_window_margin_ok(logits, eps):
            return eps
    return None


def layer0_logits(oracle, shape, h):
    norm, router, _ = U.dense(oracle, U.SEED, shape, 0)
    return oracle.gemv_f32(router, oracle.rmsnorm_1p(h, norm, shape.eps))


@pytest.mark.parametrize("kind", [U.HK_Q4, U.HK_MIXED])
def test_decode_layer_and_stack_follow_the_tie_window(ctx, oracle, kind):
    from hawking_amd.moe import MoeModel, MoeShape
    shape = MoeShape(n_layers=2, hidden=512, inter=256, shared_inter=256, n_experts=64, top_k=6, expert_kind=kind,
                     expert_group=32 if kind == U.HK_Q4 else 128)
    say("tie window, decode layer + stack", kind)
    for trial in range(16):
        h = oracle.normal(oracle.stream_key(U.SEED, 0x71E0 + trial), 512, 1.0)
        eps = discriminating_window(oracle, layer0_logits(oracle, shape, h), shape.top_k)
        if eps is not None:
            break
    else:
        pytest.fail("no input gave a discriminating tie window")
    shape.route_tie_eps = eps
    m = MoeModel(ctx, shape)
    m.fill_synthetic(U.SEED)
    ctx.device_status()
    out, ids, w = m.moe_suffix(0, h)
    L, rout, rids, rw, logits = U.oracle_layer(oracle, U.SEED, shape, 0, h)
    strict, _ = oracle.router_softmax_topk(logits, shape.top_k, 0.0)
    assert rids.tolist() != strict.tolist()
    assert ids.tolist() == rids.tolist()
    assert np.max(np.abs(w - rw)) <= 1e-6
    assert oracle.relative_l2(out, rout) < TOL
    assert oracle.relative_l2(out, L.forward_f64(h, ids)) < TOL
    # both layers through the stack: per-layer launches vs the persistent
    # launch (its route and down roles rank with the same window), same bits
    pout, pids, pw = m.forward_token(h)
    m.set_stack_launch(1)
    try:
        assert m.stack_is_persistent()
        qout, qids, qw = m.forward_token(h)
    finally:
        m.set_stack_launch(0)
    assert pids[0].tolist() == rids.tolist()
    assert np.array_equal(pids, qids) and np.array_equal(pw.view(np.uint32), qw.view(np.uint32))
    assert np.array_equal(pout.view(np.uint32), qout.view(np.uint32))
    assert ctx.device_status() == 0


def test_mixed15_layer_follows_the_tie_window(ctx, oracle):
    from hawking_amd.moe import Mixed15Layer
    from tests.test_gpu_moe15 import _key, build_layer
    H, I, SI, E, K, rank = 512, 128, 128, 64, 6, 32
    say("tie window, mixed15 layer")
    layer, ref = build_layer(ctx, oracle, H, I, SI, E, K, rank, tag=0x50)
    for trial in range(16):
        h = oracle.normal(_key(oracle, 0x51, trial), H, 1.0)
        *_, logits = ref.forward(h)
        eps = discriminating_window(oracle, logits, K)
        if eps is not None:
            break
    else:
        pytest.fail("no input gave a discriminating tie window")
    router, experts, shared, sgate = layer._keep
    tl = Mixed15Layer(ctx, ref.norm_w, router, experts, K, shared=shared, shared_gate=sgate, route_tie_eps=eps)
    tref = oracle.MoeLayer(H, I, E, K, ref.norm_w, ref.router_w, ref._experts, shared=ref._shared,
                           shared_gate_w=ref.shared_gate_w, tie_eps=eps)
    ctx.device_status()
    out, ids, w = tl.moe_suffix(h)
    rout, rids, rw, _, rlogits = tref.forward(h)
    strict, _ = oracle.router_softmax_topk(rlogits, K, 0.0)
    assert rids.tolist() != strict.tolist()
    assert ids.tolist() == rids.tolist()
    assert np.max(np.abs(w - rw)) <= 2e-6
    assert oracle.relative_l2(out, rout) < TOL
    assert oracle.relative_l2(out, tref.forward_f64(h, ids)) < TOL
    assert ctx.device_status() == 0
    tl.free()
    layer.free()
