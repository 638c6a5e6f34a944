"""GPU parity of the batched noaux_tc MoE block (routed_moe with batched_mlp,
gravity_glm.rs:447-600) against the CPU oracle.

Router ids exact under the noaux_tc margin rule, weights within 1e-6 abs,
outputs within 2e-5 rel-L2 of the oracle's f32 routed_moe and of the FP64
authority; a token's output does not depend on the rest of the batch (each
token's arithmetic is independent of how tokens are grouped by expert).
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


def _inputs(oracle, T, hidden, salt):
    x = oracle.normal(oracle.stream_key(U.SEED, 0xB5000 + salt), T * hidden, 1.0).reshape(T, hidden)
    xb = U.to_bf16_bits(x)
    return xb, U.bf16_to_f32(xb)


def _check_tokens(oracle, shape, layer, seed, x32, y, ids, w, tokens):
    checked = 0
    for t in tokens:
        M, out, rids, rw, logits = U.oracle_noaux(oracle, seed, shape, layer, x32[t])
        bias = U.router_bias(oracle, seed, shape, layer)
        if not U.noaux_margin_ok(logits, bias, shape.n_group, shape.topk_group, shape.top_k):
            continue
        checked += 1
        assert ids[t].tolist() == rids.tolist(), f"token {t}"
        assert np.max(np.abs(w[t] - rw)) <= 1e-6, f"token {t}"
        assert oracle.relative_l2(y[t], out) < TOL, f"token {t}"
        assert oracle.relative_l2(y[t], M.forward_f64(x32[t], ids[t])) < TOL, f"token {t}"
    return checked


SMALL = [
    # (label, n_group, topk_group, norm, scaling, shared_inter, T)
    ("g8t4-norm-x2.5-32tok", 8, 4, True, 2.5, 256, 32),
    ("g1t1-nonorm-5tok", 1, 1, False, 1.0, 256, 5),
    ("g4t2-noshared-64tok", 4, 2, True, 1.0, 0, 64),
]


@pytest.mark.parametrize("label,n_group,topk_group,norm,scaling,shared_inter,T", SMALL)
def test_small_block_all_tokens(ctx, oracle, label, n_group, topk_group, norm, scaling, shared_inter, T):
    from hawking_amd.moe import MoeModel, MoeShape
    shape = MoeShape(n_layers=1, hidden=512, inter=256, shared_inter=shared_inter, n_experts=64, top_k=6,
                     expert_kind=U.HK_Q4, expert_group=32, shared_gate=False, router=1, n_group=n_group,
                     topk_group=topk_group, norm_topk_prob=norm, routed_scaling_factor=scaling)
    say("batched block", label)
    m = MoeModel(ctx, shape)
    m.fill_synthetic(U.SEED + 11)
    ctx.device_status()
    xb, x32 = _inputs(oracle, T, 512, T)
    y, ids, w = m.routed_moe(0, xb)
    assert ctx.device_status() == 0
    assert _check_tokens(oracle, shape, 0, U.SEED + 11, x32, y, ids, w, range(T)) >= T // 2


def test_uploaded_block_matches_oracle(ctx, oracle):
    """Weights uploaded from host canonical arrays (set_layer), not generated."""
    from hawking_amd.moe import MoeModel, MoeShape
    shape = MoeShape(n_layers=1, hidden=256, inter=128, shared_inter=128, n_experts=16, top_k=4,
                     expert_kind=U.HK_Q4, expert_group=64, shared_gate=False, router=1, n_group=4, topk_group=2,
                     norm_topk_prob=True, routed_scaling_factor=2.5)
    say("uploaded batched block")
    seed = 5
    experts = [tuple(U.oracle_organ(oracle, seed, shape, 0, e, p) for p in range(3)) for e in range(16)]
    shared = tuple(U.oracle_organ(oracle, seed, shape, 0, 16, p) for p in range(3))
    norm, router, _ = U.dense(oracle, seed, shape, 0)
    bias = U.router_bias(oracle, seed, shape, 0)
    M = oracle.NoauxMoe(256, 16, 4, 4, 2, True, 2.5, router, bias, experts, shared)
    m = MoeModel(ctx, shape)
    m.set_layer(0, norm, router, [tuple(U.organ_dict(o) for o in t) for t in experts],
                shared=[U.organ_dict(o) for o in shared], router_bias=bias)
    xb, x32 = _inputs(oracle, 12, 256, 7)
    y, ids, w = m.routed_moe(0, xb)
    for t in range(12):
        out, rids, rw, logits = M.forward(x32[t])
        if not U.noaux_margin_ok(logits, bias, 4, 2, 4):
            continue
        assert ids[t].tolist() == rids.tolist()
        assert np.max(np.abs(w[t] - rw)) <= 1e-6
        assert oracle.relative_l2(y[t], out) < TOL
        assert oracle.relative_l2(y[t], M.forward_f64(x32[t], ids[t])) < TOL


def test_config5_deepseek_v3_block(ctx, oracle):
    """Config 5 at full size: hidden 7168, 256 experts x 2048 (Q4 G32) + shared,
    top-8 noaux_tc, 32 bf16 tokens.  Every token's route against the oracle's
    noaux_tc on the oracle's router logits (ids exact under the margin rule,
    weights within 1e-6); four tokens' outputs against the oracle's routed_moe
    and the FP64 authority (experts generated once and shared between them);
    three tokens against their own batch-of-one run (bit-identical)."""
    import concurrent.futures as cf
    from hawking_amd.moe import MoeModel, MoeShape
    shape = MoeShape.deepseek_v3()
    say("config5 full block, 32 tokens")
    m = MoeModel(ctx, shape)
    m.fill_synthetic(U.SEED)
    xb, x32 = _inputs(oracle, 32, 7168, 5)
    y, ids, w = m.routed_moe(0, xb)
    assert ctx.device_status() == 0
    for t in range(32):
        assert len(set(ids[t].tolist())) == 8
    for t in (0, 17, 31):
        y1, ids1, w1 = m.routed_moe(0, xb[t:t + 1])
        assert np.array_equal(ids1[0], ids[t]) and np.array_equal(w1[0], w[t])
        assert np.array_equal(y1[0], y[t]), f"token {t} depends on the batch"
    say("config5 routes of all 32 tokens vs the oracle")
    _, router, _ = U.dense(oracle, U.SEED, shape, 0)
    bias = U.router_bias(oracle, U.SEED, shape, 0)
    routed = 0
    for t in range(32):
        logits = oracle.gemv_f32(router, x32[t])
        if not U.noaux_margin_ok(logits, bias, shape.n_group, shape.topk_group, shape.top_k):
            continue
        rids, rw = oracle.router_noaux_tc(logits, bias, shape.n_group, shape.topk_group, shape.top_k,
                                          shape.norm_topk_prob, shape.routed_scaling_factor)
        assert ids[t].tolist() == rids.tolist(), f"token {t}"
        assert np.max(np.abs(w[t] - rw)) <= 1e-6, f"token {t}"
        routed += 1
    assert routed >= 28, f"only {routed} of 32 tokens passed the margin rule"
    say("config5 outputs of four tokens vs the oracle")
    cache = {}
    shared = tuple(U.oracle_organ(oracle, U.SEED, shape, 0, shape.n_experts, p) for p in range(3))
    checked = 0
    with cf.ThreadPoolExecutor(max_workers=8) as pool:
        for t in (0, 9, 22, 31):
            logits = oracle.gemv_f32(router, x32[t])
            if not U.noaux_margin_ok(logits, bias, shape.n_group, shape.topk_group, shape.top_k):
                continue
            want = [int(e) for e in ids[t] if int(e) not in cache]
            made = list(pool.map(lambda ep: U.oracle_organ(oracle, U.SEED, shape, 0, ep[0], ep[1]),
                                 [(e, p) for e in want for p in range(3)]))
            for i, e in enumerate(want):
                cache[e] = tuple(made[3 * i:3 * i + 3])
            experts = [None] * shape.n_experts
            for e in ids[t].tolist():
                experts[e] = cache[e]
            M = oracle.NoauxMoe(shape.hidden, shape.n_experts, shape.top_k, shape.n_group, shape.topk_group,
                                shape.norm_topk_prob, shape.routed_scaling_factor, router, bias, experts, shared)
            out, rids, rw, _ = M.forward(x32[t])
            assert ids[t].tolist() == rids.tolist(), f"token {t}"
            assert oracle.relative_l2(y[t], out) < TOL, f"token {t}"
            assert oracle.relative_l2(y[t], M.forward_f64(x32[t], ids[t])) < TOL, f"token {t}"
            checked += 1
    assert checked >= 3


def test_batch_rejects_bad_calls(ctx):
    from hawking_amd._lib import HK_E_INVALID_ARG, HK_E_UNSUPPORTED, HawkingError
    from hawking_amd.moe import MoeModel, MoeShape
    q = MoeModel(ctx, MoeShape(n_layers=1, hidden=256, inter=128, shared_inter=128, n_experts=16, top_k=4,
                               expert_kind=U.HK_Q4, expert_group=32))
    q.fill_synthetic(1)
    with pytest.raises(HawkingError) as e:
        q.routed_moe(0, np.zeros((2, 256), np.uint16))
    assert e.value.code == HK_E_UNSUPPORTED  # softmax-routed model has no batched block
    b = MoeModel(ctx, MoeShape(n_layers=1, hidden=256, inter=128, shared_inter=128, n_experts=16, top_k=4,
                               expert_kind=U.HK_Q4, expert_group=32, shared_gate=False, router=1, n_group=4,
                               topk_group=2))
    b.fill_synthetic(1)
    with pytest.raises(HawkingError) as e:
        b.routed_moe(0, np.zeros((65, 256), np.uint16))
    assert e.value.code == HK_E_INVALID_ARG
    with pytest.raises(HawkingError) as e:
        b.decode_layer_device(0, ctx.empty(256), ctx.empty(256))
    assert e.value.code == HK_E_UNSUPPORTED
