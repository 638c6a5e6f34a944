"""GPU parity of the routers and the MoE decode step against the CPU oracle.

Router ids must match exactly (planted ties from the reference's
moe_topk_gate_exact_ties_parity.rs, and random logits under the router
margin rule); weights within 1e-6 abs; layer outputs within 2e-5 rel-L2 of
the oracle's moe_suffix and of the FP64 authority.
"""
import sys

import numpy as np
import pytest

from tests import hk_testutil as U
from tests.test_oracle_router_moe import TIE_CASES

pytestmark = pytest.mark.gpu
TOL = 2e-5


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    from hawking_amd.runtime import Context
    return Context(0)


# ------------------------------------------------------------------ routers

@pytest.mark.parametrize("label,make,k,want", TIE_CASES)
def test_router_exact_tie_fixtures(ctx, oracle, label, make, k, want):
    from hawking_amd.moe import topk_router
    logits = make()
    say("router ties", label)
    ids, w = topk_router(ctx, logits, k, renorm=False)
    sids, sw = oracle.topk_softmax_batch(logits, 1, logits.size, k)
    assert ids[0].tolist() == want == sids.tolist()
    assert np.max(np.abs(w[0] - sw)) <= 1e-5
    ids, w = topk_router(ctx, logits, k, renorm=True)
    rids, rw = oracle.router_softmax_topk(logits, k)
    assert ids[0].tolist() == rids.tolist()
    assert np.max(np.abs(w[0] - rw)) <= 1e-6


def test_router_random_batch_under_margin_rule(ctx, oracle):
    from hawking_amd.moe import topk_router
    rng = np.random.default_rng(5)
    n_tok, E, k = 64, 512, 10
    logits = (rng.standard_normal((n_tok, E)) * 0.7).astype(np.float32)
    say("router batch", n_tok, E, k)
    ids, w = topk_router(ctx, logits, k, n_tokens=n_tok)
    checked = 0
    for t in range(n_tok):
        if not U.router_margin_ok(logits[t], k):
            continue
        rids, rw = oracle.router_softmax_topk(logits[t], k)
        assert ids[t].tolist() == rids.tolist()
        assert np.max(np.abs(w[t] - rw)) <= 1e-6
        checked += 1
    assert checked > n_tok // 2


def test_router_tie_eps_window_is_serial_rule(ctx, oracle):
    from hawking_amd.moe import topk_router
    logits = np.full(32, -2.0, np.float32)
    logits[[3, 9, 17]] = [1.0, 1.0 + 1e-4, 1.0 + 3e-4]
    eps = 2e-5
    say("router tie_eps")
    ids, w = topk_router(ctx, logits, 3, tie_eps=eps)
    rids, rw = oracle.router_softmax_topk(logits, 3, eps)
    assert ids[0].tolist() == rids.tolist()


def test_noaux_tc_matches_oracle(ctx, oracle):
    from hawking_amd.moe import noaux_tc_router
    rng = np.random.default_rng(6)
    n_tok, E = 32, 256
    logits = rng.standard_normal((n_tok, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)
    for (ng, tg) in [(1, 1), (8, 4)]:
        say("noaux_tc", ng, tg)
        ids, w = noaux_tc_router(ctx, logits, bias, ng, tg, 8, True, 2.5, n_tokens=n_tok)
        for t in range(n_tok):
            rids, rw = oracle.router_noaux_tc(logits[t], bias, ng, tg, 8, True, 2.5)
            assert ids[t].tolist() == rids.tolist()
            assert np.max(np.abs(w[t] - rw)) <= 1e-5


def test_router_rejects_bad_geometry(ctx):
    from hawking_amd._lib import HK_E_INVALID_ARG, HawkingError
    from hawking_amd.moe import topk_router
    from hawking_amd._lib import HK_E_UNSUPPORTED
    with pytest.raises(HawkingError) as e:
        topk_router(ctx, np.zeros(8, np.float32), 9)
    assert e.value.code == HK_E_INVALID_ARG
    with pytest.raises(HawkingError) as e:
        topk_router(ctx, np.zeros(128, np.float32), 65)
    assert e.value.code == HK_E_UNSUPPORTED


def test_router_flags_nonfinite_logits(ctx):
    from hawking_amd.moe import topk_router
    ctx.device_status()  # clear
    logits = np.zeros(16, np.float32)
    logits[4] = np.inf
    topk_router(ctx, logits, 2)
    assert ctx.device_status() & 1


# ------------------------------------------------------------------ MoE layer

def _small_model(ctx, oracle, kind):
    from hawking_amd.moe import MoeModel, MoeShape
    shape = MoeShape(n_layers=1, hidden=256, inter=128, shared_inter=128, n_experts=16, top_k=4,
                     expert_kind=kind, expert_group=32 if kind == U.HK_Q4 else 128)
    seed = 99
    experts = [tuple(U.oracle_organ(oracle, seed, shape, 0, e, p) for p in range(3)) for e in range(16)]
    shared = tuple(U.oracle_organ(oracle, seed, shape, 0, 16, p) for p in range(3))
    norm, router, gate = U.dense(oracle, seed, shape, 0)
    L = oracle.MoeLayer(256, 128, 16, 4, norm, router, experts, shared=shared, shared_gate_w=gate)
    m = MoeModel(ctx, shape)
    m.set_layer(0, norm, router, [tuple(U.organ_dict(o) for o in t) for t in experts],
                shared=[U.organ_dict(o) for o in shared], shared_gate_w=gate)
    return m, L, shape


@pytest.mark.parametrize("kind", [U.HK_Q4, U.HK_MIXED])
def test_small_layer_uploaded_from_oracle(ctx, oracle, kind):
    say("small layer", kind)
    m, L, shape = _small_model(ctx, oracle, kind)
    rng = np.random.default_rng(kind)
    for trial in range(4):
        h = rng.standard_normal(256).astype(np.float32)
        out, ids, w = m.moe_suffix(0, h)
        rout, rids, rw, _, logits = L.forward(h)
        if U.router_margin_ok(logits, 4):
            assert ids.tolist() == rids.tolist()
            assert np.max(np.abs(w - rw)) <= 1e-6
        assert oracle.relative_l2(out, rout) < TOL
        assert oracle.relative_l2(out, L.forward_f64(h, ids)) < TOL


def test_decode_router_exact_ties_and_flat_logits(ctx, oracle):
    """The decode top-k (threshold + rank, k-round fallback past 64
    candidates) on exact ties: duplicated router rows give equal logits,
    ranked by index; all-zero router rows give 128 equal probabilities (the
    fallback), so the route is experts 0..k-1 with weight 1/k each."""
    from hawking_amd.moe import MoeModel, MoeShape
    E, K = 128, 8
    shape = MoeShape(n_layers=1, hidden=256, inter=128, shared_inter=128, n_experts=E, top_k=K,
                     expert_kind=U.HK_Q4, expert_group=32)
    seed = 77
    experts = [tuple(U.oracle_organ(oracle, seed, shape, 0, e, p) for p in range(3)) for e in range(E)]
    shared = tuple(U.oracle_organ(oracle, seed, shape, 0, E, p) for p in range(3))
    norm, router, gate = U.dense(oracle, seed, shape, 0)
    h = oracle.normal(oracle.stream_key(U.SEED, 0x71E), 256, 1.0)
    logits = oracle.MoeLayer(256, 128, E, K, norm, router, experts, shared=shared, shared_gate_w=gate).forward(h)[4]
    top = int(np.argmax(logits))
    tied = router.copy()
    for e in (5, 40, 77, 100):      # four equal logits, twice the largest
        tied[e] = 2.0 * router[top]
    for e in (9, 10):               # two more equal ones
        tied[e] = 1.5 * router[top]
    m = MoeModel(ctx, shape)
    for label, R in (("tied rows", tied), ("flat", np.zeros_like(router))):
        say("decode router", label)
        m.set_layer(0, norm, R, [tuple(U.organ_dict(o) for o in t) for t in experts],
                    shared=[U.organ_dict(o) for o in shared], shared_gate_w=gate)
        L = oracle.MoeLayer(256, 128, E, K, norm, R, experts, shared=shared, shared_gate_w=gate)
        out, ids, w = m.moe_suffix(0, h)
        rout, rids, rw, _, logits = L.forward(h)
        assert ids.tolist() == rids.tolist(), label
        assert np.max(np.abs(w - rw)) <= 1e-6
        assert oracle.relative_l2(out, rout) < TOL
        if label == "flat":
            assert ids.tolist() == list(range(K))
            assert np.allclose(w, 1.0 / K, rtol=0, atol=1e-7)
        else:
            pos = [ids.tolist().index(e) for e in (5, 40, 77, 100)]
            assert pos == sorted(pos)


def test_decode_router_nan_logit_leaves_no_unset_slot(ctx, oracle):
    """One NaN router logit (a NaN in one router row): the status bit is set,
    and every published route slot is a valid distinct id or -1 with weight
    0 -- never an unset slot (a NaN probability is never a candidate, so
    fewer than k candidates can remain)."""
    from hawking_amd.moe import MoeModel, MoeShape
    E, K = 64, 8
    shape = MoeShape(n_layers=1, hidden=256, inter=128, shared_inter=128, n_experts=E, top_k=K,
                     expert_kind=U.HK_Q4, expert_group=32)
    seed = 78
    experts = [tuple(U.oracle_organ(oracle, seed, shape, 0, e, p) for p in range(3)) for e in range(E)]
    shared = tuple(U.oracle_organ(oracle, seed, shape, 0, E, p) for p in range(3))
    norm, router, gate = U.dense(oracle, seed, shape, 0)
    h = oracle.normal(oracle.stream_key(U.SEED, 0x7A7), 256, 1.0)
    m = MoeModel(ctx, shape)
    for label, rows in (("one NaN row", [9]), ("all NaN", list(range(E)))):
        say("decode router", label)
        R = router.copy()
        R[rows, 3] = np.nan
        m.set_layer(0, norm, R, [tuple(U.organ_dict(o) for o in t) for t in experts],
                    shared=[U.organ_dict(o) for o in shared], shared_gate_w=gate)
        ctx.device_status()
        out, ids, w = m.moe_suffix(0, h)
        assert ctx.device_status() & 1
        valid = [int(i) for i in ids if i >= 0]
        assert all(i < E for i in valid) and len(set(valid)) == len(valid)
        assert all((i >= 0) or (wt == 0.0) for i, wt in zip(ids.tolist(), w.tolist()))
        assert set(ids.tolist()) <= set(range(E)) | {-1}


@pytest.mark.parametrize("kind", [U.HK_Q4, U.HK_MIXED])
def test_synthetic_layer_matches_oracle_regeneration(ctx, oracle, kind):
    """Device-generated weights == oracle-regenerated weights, end to end."""
    from hawking_amd.moe import MoeModel, MoeShape
    shape = MoeShape(n_layers=2, hidden=512, inter=256, shared_inter=256, n_experts=64, top_k=6,
                     expert_kind=kind, expert_group=32 if kind == U.HK_Q4 else 128)
    say("synthetic layer", kind)
    m = MoeModel(ctx, shape)
    m.fill_synthetic(U.SEED)
    h = oracle.normal(oracle.stream_key(U.SEED, 0xF00D), 512, 1.0)
    for layer in range(2):
        out, ids, w = m.moe_suffix(layer, h)
        L, rout, rids, rw, logits = U.oracle_layer(oracle, U.SEED, shape, layer, h)
        assert U.router_margin_ok(logits, shape.top_k)
        assert ids.tolist() == rids.tolist()
        assert np.max(np.abs(w - rw)) <= 1e-6
        assert oracle.relative_l2(out, rout) < TOL
        assert oracle.relative_l2(out, L.forward_f64(h, ids)) < TOL
        for e in ids.tolist()[:2]:
            o = U.oracle_organ(oracle, U.SEED, shape, layer, e, 0)
            want = (o.scales.nbytes + o.codes.nbytes) if kind == U.HK_Q4 else o.mixed.nbytes()
            assert m.expert_bytes(layer, e) >= want


VARIANTS = [
    # (label, kind, group, inter, shared_inter, shared_gate)
    ("q4-g64-wide-shared", U.HK_Q4, 64, 128, 256, True),
    ("q4-g128-no-shared", U.HK_Q4, 128, 256, 0, False),
    ("mixed-shared-no-gate", U.HK_MIXED, 128, 256, 256, False),
    ("mixed-inter384-narrow-shared", U.HK_MIXED, 128, 384, 128, True),
    # routed and shared down organs with different numbers of 512-column steps
    # (the down kernel reads each slot's copied step headers at its own stride)
    ("mixed-inter512-shared1024", U.HK_MIXED, 128, 512, 1024, True),
    ("mixed-inter1024-shared512", U.HK_MIXED, 128, 1024, 512, True),
]


@pytest.mark.parametrize("label,kind,group,inter,shared_inter,shared_gate", VARIANTS)
def test_synthetic_layer_variants(ctx, oracle, label, kind, group, inter, shared_inter, shared_gate):
    """Group sizes, no shared expert, a shared expert of another width, an
    ungated shared expert, and an intermediate that is not a whole number of
    512-column steps."""
    from hawking_amd.moe import MoeModel, MoeShape
    shape = MoeShape(n_layers=1, hidden=512, inter=inter, shared_inter=shared_inter, n_experts=32, top_k=5,
                     expert_kind=kind, expert_group=group, shared_gate=shared_gate)
    say("layer variant", label)
    m = MoeModel(ctx, shape)
    m.fill_synthetic(U.SEED + 7)
    ctx.device_status()  # clear
    checked = 0
    for trial in range(3):
        h = oracle.normal(oracle.stream_key(U.SEED, 0xBEEF + trial), 512, 1.0)
        out, ids, w = m.moe_suffix(0, h)
        L, rout, rids, rw, logits = U.oracle_layer(oracle, U.SEED + 7, shape, 0, h)
        if not U.router_margin_ok(logits, shape.top_k):
            continue
        checked += 1
        assert ids.tolist() == rids.tolist()
        assert np.max(np.abs(w - rw)) <= 1e-6
        assert oracle.relative_l2(out, rout) < TOL
        assert oracle.relative_l2(out, L.forward_f64(h, ids)) < TOL
    assert checked >= 1
    assert ctx.device_status() == 0


def test_layer_flags_nonfinite_hidden_state(ctx, oracle):
    """A NaN in h is latched in the device status word; every kernel still
    ends normally and the next clean call is exact again."""
    from hawking_amd.moe import MoeModel, MoeShape
    shape = MoeShape(n_layers=1, hidden=256, inter=128, shared_inter=128, n_experts=16, top_k=4,
                     expert_kind=U.HK_Q4, expert_group=32)
    say("non-finite hidden state")
    m = MoeModel(ctx, shape)
    m.fill_synthetic(U.SEED)
    ctx.device_status()  # clear
    h = np.ones(256, np.float32)
    h[3] = np.nan
    m.moe_suffix(0, h)
    assert ctx.device_status() != 0
    h = oracle.normal(oracle.stream_key(U.SEED, 0xAB), 256, 1.0)
    out, ids, w = m.moe_suffix(0, h)
    L, rout, rids, rw, logits = U.oracle_layer(oracle, U.SEED, shape, 0, h)
    assert ctx.device_status() == 0
    if U.router_margin_ok(logits, shape.top_k):
        assert ids.tolist() == rids.tolist()
    assert oracle.relative_l2(out, L.forward_f64(h, ids)) < TOL


def test_config3_qwen3next_layer_full_size(ctx, oracle):
    """Config 3: hidden 2048, 512 experts x inter 512 (Q4 G32) + shared, top-10."""
    from hawking_amd.moe import MoeModel, MoeShape
    shape = MoeShape(n_layers=1, hidden=2048, inter=512, shared_inter=512, n_experts=512, top_k=10,
                     expert_kind=U.HK_Q4, expert_group=32)
    say("config3 full layer")
    m = MoeModel(ctx, shape)
    m.fill_synthetic(U.SEED)
    h = oracle.normal(oracle.stream_key(U.SEED, 0xC3), 2048, 1.0)
    out, ids, w = m.moe_suffix(0, h)
    L, rout, rids, rw, logits = U.oracle_layer(oracle, U.SEED, shape, 0, h)
    assert U.router_margin_ok(logits, 10)
    assert ids.tolist() == rids.tolist()
    assert np.max(np.abs(w - rw)) <= 1e-6
    assert oracle.relative_l2(out, rout) < TOL
    assert oracle.relative_l2(out, L.forward_f64(h, ids)) < TOL


def test_stack_matches_oracle_layer_by_layer(ctx, oracle):
    """Config 4 geometry (mixed <=1.5 BPW, Qwen3-Next layer) over 3 layers."""
    from hawking_amd.moe import MoeModel, MoeShape
    shape = MoeShape(n_layers=3, hidden=2048, inter=512, shared_inter=512, n_experts=512, top_k=10,
                     expert_kind=U.HK_MIXED, expert_group=128)
    say("config4 geometry, 3 layers")
    m = MoeModel(ctx, shape)
    m.fill_synthetic(U.SEED)
    h0 = oracle.normal(oracle.stream_key(U.SEED, 0xC4), 2048, 1.0)
    out, ids, w = m.forward_token(h0)
    h = h0
    for layer in range(3):
        L, h_next, rids, rw, logits = U.oracle_layer(oracle, U.SEED, shape, layer, h)
        assert U.router_margin_ok(logits, 10), f"near-tie at layer {layer}"
        assert ids[layer].tolist() == rids.tolist()
        h = h_next
    assert oracle.relative_l2(out, h) < TOL
