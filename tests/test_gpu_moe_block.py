"""GPU parity of hk_moe_block, the BackendMoe::moe_block seam
(crates/hawking-core/src/backend/mod.rs:509-521): the routed (and optional
shared) expert block for CALLER-supplied device routes, accumulated into
out.  Routes come from the oracle's router; the expert block is checked
against the oracle's moe_suffix (out = h), its FP64 authority, and the
routed-only weighted sum of run_qwen80_routed_expert_table
(model/qwen80_device_expert_table.rs:1204-1247), within 2e-5 relative L2.
"""
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


def _small(ctx, oracle, kind, seed=123):
    from hawking_amd.moe import MoeModel, MoeShape
    shape = MoeShape(n_layers=1, hidden=256, inter=128, shared_inter=128, n_experts=16, top_k=4,
                     expert_kind=kind, expert_group=32 if kind == U.HK_Q4 else 128)
    experts = [tuple(U.oracle_organ(oracle, seed, shape, 0, e, p) for p in range(3)) for e in range(16)]
    shared = tuple(U.oracle_organ(oracle, seed, shape, 0, 16, p) for p in range(3))
    norm, router, gate = U.dense(oracle, seed, shape, 0)
    L = oracle.MoeLayer(256, 128, 16, 4, norm, router, experts, shared=shared, shared_gate_w=gate)
    m = MoeModel(ctx, shape)
    m.set_layer(0, norm, router, [tuple(U.organ_dict(o) for o in t) for t in experts],
                shared=[U.organ_dict(o) for o in shared], shared_gate_w=gate)
    return m, L, experts, shared, gate


def routed_sum(oracle, experts, ids, w, x):
    """sum_r w_r down(silu(gate x) * up x), route order, serial f32."""
    comb = np.zeros(experts[ids[0]][2].rows, np.float32)
    for e, wr in zip(ids, w):
        g, u, d = experts[e]
        y = d.matvec(oracle.silu_mul(g.matvec(x), u.matvec(x)))
        comb = (comb + np.float32(wr) * y).astype(np.float32)
    return comb


@pytest.mark.parametrize("kind", [U.HK_Q4, U.HK_MIXED])
def test_block_with_oracle_routes_is_moe_suffix(ctx, oracle, kind):
    say("moe_block = moe_suffix with caller routes", kind)
    m, L, experts, shared, gate = _small(ctx, oracle, kind)
    rng = np.random.default_rng(40 + kind)
    ctx.device_status()
    for trial in range(3):
        h = rng.standard_normal(256).astype(np.float32)
        rout, rids, rw, xn, logits = L.forward(h)
        out = m.moe_block(0, rids, rw, xn, out=h)
        assert oracle.relative_l2(out, rout) < TOL
        assert oracle.relative_l2(out, L.forward_f64(h, rids)) < TOL
    assert ctx.device_status() == 0


@pytest.mark.parametrize("kind", [U.HK_Q4, U.HK_MIXED])
def test_block_routed_only_and_partial_routes(ctx, oracle, kind):
    """include_shared = 0 and out = 0 is the expert table's combined; fewer
    routes than top_k, and weights that do not sum to one, are taken as given."""
    say("moe_block routed only", kind)
    m, L, experts, shared, gate = _small(ctx, oracle, kind)
    x = oracle.normal(oracle.stream_key(U.SEED, 0xB10C + kind), 256, 1.0)
    for ids, w in (([3, 11, 0, 7], [0.4, 0.3, 0.2, 0.1]), ([15, 2], [0.9, -0.25]), ([5], [1.0])):
        got = m.moe_block(0, ids, w, x, include_shared=False)
        want = routed_sum(oracle, experts, ids, np.asarray(w, np.float32), x)
        assert oracle.relative_l2(got, want) < TOL, (ids, w)


def test_block_in_place_and_invalid_route(ctx, oracle):
    """x and out may be one vector; an id outside [0, n_experts) adds nothing
    and latches the route bit."""
    say("moe_block in place, invalid id")
    m, L, experts, shared, gate = _small(ctx, oracle, U.HK_Q4)
    x = oracle.normal(oracle.stream_key(U.SEED, 0xB10D), 256, 1.0)
    ids = np.array([1, 999, 6], np.int32)
    w = np.array([0.5, 0.3, 0.2], np.float32)
    ctx.device_status()
    xd = ctx.to_device(x)
    m.moe_block_device(0, ctx.to_device(ids), ctx.to_device(w), 3, xd, xd, include_shared=False)
    got = xd.download()
    assert ctx.device_status() & 2
    want = (x + routed_sum(oracle, experts, [1, 6], w[[0, 2]], x)).astype(np.float32)
    assert oracle.relative_l2(got, want) < TOL


def test_block_rejects_bad_arguments(ctx, oracle):
    from hawking_amd._lib import HK_E_INVALID_ARG, HawkingError
    m, L, experts, shared, gate = _small(ctx, oracle, U.HK_Q4)
    x = np.zeros(256, np.float32)
    with pytest.raises(HawkingError) as e:
        m.moe_block(0, [0, 1, 2, 3, 4], [0.2] * 5, x)   # more routes than top_k
    assert e.value.code == HK_E_INVALID_ARG


def test_block_config3_full_size(ctx, oracle):
    """Config 3 (hidden 2048, 512 experts x inter 512, Q4 G32, shared + gate):
    RMSNorm and router on the oracle, the expert block on the device with the
    oracle's route, out = h."""
    from hawking_amd.moe import MoeModel, MoeShape
    shape = MoeShape(n_layers=1, hidden=2048, inter=512, shared_inter=512, n_experts=512, top_k=10,
                     expert_kind=U.HK_Q4, expert_group=32)
    say("moe_block config3")
    m = MoeModel(ctx, shape)
    m.fill_synthetic(U.SEED)
    h = oracle.normal(oracle.stream_key(U.SEED, 0xC3B), 2048, 1.0)
    L, rout, rids, rw, logits = U.oracle_layer(oracle, U.SEED, shape, 0, h)
    norm, _, _ = U.dense(oracle, U.SEED, shape, 0)
    xn = oracle.rmsnorm_1p(h, norm, shape.eps)
    out = m.moe_block(0, rids, rw, xn, out=h)
    assert oracle.relative_l2(out, rout) < TOL
    assert oracle.relative_l2(out, L.forward_f64(h, rids)) < TOL
