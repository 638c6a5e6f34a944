"""Pin the oracle's router, activations and MoE layer.

Known answers come from the reference's own tests:
  * crates/hawking-core/tests/moe_topk_gate_exact_ties_parity.rs:76-155 (planted ties)
  * crates/hawking-core/src/moe.rs:143-155 (topk_picks_largest)
  * crates/hawking-core/src/gravity_glm.rs:3664-3667 (topk_desc ties -> lower index)
The layer itself is checked against its FP64 authority and against closed
forms (zero experts, identical experts, top_k = n_experts).
"""
import numpy as np
import pytest


def _tie_fixture_boundary():
    logits = np.full(128, -3.0, np.float32)
    logits[:12] = 5.0
    logits[20:28] = 1.0
    logits[40] = 2.0
    for i in range(50, 128):
        logits[i] = -1.0 - (i % 17) * 0.01
    return logits


def _tie_fixture_interior():
    logits = np.full(128, -4.0, np.float32)
    for rank, idx in enumerate([90, 10, 50, 3, 70]):
        logits[idx] = 10.0 - rank
    for idx in (100, 25, 110, 15):
        logits[idx] = 4.0
    return logits


TIE_CASES = [
    ("boundary-ties-128x8", _tie_fixture_boundary, 8, list(range(8))),
    ("interior-ties-128x8", _tie_fixture_interior, 8, [90, 10, 50, 3, 70, 15, 25, 100]),
    ("all-equal-64x6", lambda: np.full(64, 0.25, np.float32), 6, list(range(6))),
]


@pytest.mark.parametrize("label,make,k,want", TIE_CASES)
def test_reference_tie_fixtures(oracle, label, make, k, want):
    logits = make()
    ids, w = oracle.topk_softmax_batch(logits, 1, logits.size, k)
    assert ids.tolist() == want, label
    ids2, w2 = oracle.router_softmax_topk(logits, k)
    assert ids2.tolist() == want, label
    assert abs(float(w2.sum()) - 1.0) < 1e-4


def test_no_ties_randomish_is_sorted_prefix(oracle):
    n = 128
    logits = np.array([((i * 37 + 11) % n) / n * 12.0 - 6.0 for i in range(n)], np.float32)
    ids, _ = oracle.topk_softmax_batch(logits, 1, n, 8)
    assert ids.tolist() == np.argsort(-logits.astype(np.float64), kind="stable")[:8].tolist()


def test_topk_picks_largest(oracle):
    ids, w = oracle.router_softmax_topk(np.array([0.1, 5.0, 2.0, 0.5], np.float32), 2)
    assert ids.tolist() == [1, 2]
    assert abs(float(w.sum()) - 1.0) < 1e-5
    # closed form: renormalised softmax over the pair = sigmoid of the logit gap
    assert abs(float(w[0]) - 1.0 / (1.0 + np.exp(-3.0))) < 1e-6


def test_topk_desc_ties_lower_index_and_neg_inf(oracle):
    v = np.array([1.0, 3.0, 3.0, -np.inf, 2.0, 3.0, -np.inf], np.float32)
    assert oracle.topk_desc(v, 7).tolist() == [1, 2, 5, 4, 0, 3, 6]


def test_router_tie_window_known_answer(oracle):
    """route_tie_epsilon (src/moe.rs:8-14) in source_qwen80_topk_router
    (qwen80_complete_runtime.rs:5988-6000), derived by hand: probabilities
    q = [a, a, .20, a, a, .205, a, .22, a, .215] (a = .16 / 6) and eps = .01.
    Scanning left to right, a later q replaces the best only when it is above
    it by more than eps:
      route 0: 0 -> 2 (.20 - a > eps) -> 5 is within eps of .20 (kept 2)
               -> 7 (.22 - .20 > eps); 9 is below .22           => 7
      route 1: 0 -> 2 -> 9 (.215 - .20 = .015 > eps)              => 9
      route 2: 0 -> 2; 5 (.005 above 2) is within eps            => 2
      route 3: 0 -> 5 (the a's tie each other)                    => 5
    The strict rule (eps = 0) orders by value instead: 7, 9, 5, 2."""
    a = 0.16 / 6
    q = np.array([a, a, 0.20, a, a, 0.205, a, 0.22, a, 0.215])
    logits = np.log(q).astype(np.float32)
    ids, w = oracle.router_softmax_topk(logits, 4, 0.01)
    assert ids.tolist() == [7, 9, 2, 5]
    sel = q[[7, 9, 2, 5]] / q[[7, 9, 2, 5]].sum()
    assert np.max(np.abs(w - sel)) < 1e-6
    ids0, _ = oracle.router_softmax_topk(logits, 4, 0.0)
    assert ids0.tolist() == [7, 9, 5, 2]
    # a window narrower than every gap is the strict rule
    ids1, _ = oracle.router_softmax_topk(logits, 4, 1e-4)
    assert ids1.tolist() == [7, 9, 5, 2]


def test_router_weights_vs_f64_softmax(oracle):
    rng = np.random.default_rng(3)
    logits = (rng.standard_normal(512) * 0.5).astype(np.float32)
    ids, w = oracle.router_softmax_topk(logits, 10)
    l64 = logits.astype(np.float64)
    p = np.exp(l64 - l64.max())
    p /= p.sum()
    assert ids.tolist() == np.argsort(-p, kind="stable")[:10].tolist()
    sel = p[ids] / p[ids].sum()
    assert np.max(np.abs(w - sel)) < 1e-6


def test_router_rejects_nonfinite(oracle):
    logits = np.zeros(16, np.float32)
    logits[3] = np.nan
    with pytest.raises(oracle.OracleError):
        oracle.router_softmax_topk(logits, 4)


def test_noaux_tc_single_group_reduces_to_sorted_corrected_scores(oracle):
    rng = np.random.default_rng(4)
    logits = rng.standard_normal(256).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.01).astype(np.float32)
    ids, w = oracle.router_noaux_tc(logits, bias, 1, 1, 8, True, 2.5)
    s = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    corr = s + bias
    assert ids.tolist() == np.argsort(-corr, kind="stable")[:8].tolist()
    want = s[ids] / (s[ids].sum() + 1e-20) * 2.5
    assert np.max(np.abs(w - want)) < 1e-6


def test_noaux_tc_group_restriction_known_answer(oracle):
    # 4 groups x 4 experts; group score = sum of its best two corrected scores.
    # Group 0 has one huge expert but a weak second; groups 1 and 2 win on
    # their top-2 sums, so expert 0 is excluded although it is the maximum.
    logits = np.full(16, -6.0, np.float32)
    logits[0] = 6.0                        # group 0: 0.9975 + ~0.0025
    logits[4:6] = [2.0, 2.0]               # group 1: 0.88 + 0.88
    logits[8:10] = [1.0, 1.5]              # group 2: 0.73 + 0.82
    bias = np.zeros(16, np.float32)
    ids, w = oracle.router_noaux_tc(logits, bias, 4, 2, 3, False, 1.0)
    assert ids.tolist() == [4, 5, 9]
    assert abs(float(w[0]) - 1 / (1 + np.exp(-2.0))) < 1e-7


def test_rmsnorm_closed_form(oracle):
    x = np.array([3.0, 4.0], np.float32)
    w = np.array([0.0, 1.0], np.float32)
    out = oracle.rmsnorm_1p(x, w, 1e-6)
    inv = 1.0 / np.sqrt((9 + 16) / 2 + 1e-6)
    assert np.allclose(out, [3 * inv, 4 * inv * 2], rtol=1e-6)


def test_silu_mul_closed_form(oracle):
    g = np.array([0.0, 1.0, -2.0], np.float32)
    u = np.array([5.0, 2.0, 1.0], np.float32)
    got = oracle.silu_mul(g, u)
    want = g / (1 + np.exp(-g.astype(np.float64))) * u
    assert got[0] == 0.0 and np.allclose(got, want, rtol=1e-6)


# ------------------------------------------------------------------ MoE layer

def _small_layer(oracle, kind="q4", hidden=256, inter=128, n_experts=16, top_k=4, seed=0,
                 shared_gate=True, zero_experts=False, identical=False):
    rng = np.random.default_rng(seed)

    def organ(rows, cols):
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        if zero_experts:
            w[:] = 0
        if kind == "q4":
            return oracle.Organ.q4(w, 32), w
        sel = (rng.random(rows * cols // 128) < 0.7).astype(np.uint8)
        return oracle.Organ.mixed_from(w, sel), w

    experts = []
    first = None
    for e in range(n_experts):
        if identical and first is not None:
            experts.append(first)
            continue
        trip = tuple(organ(*s)[0] for s in [(inter, hidden), (inter, hidden), (hidden, inter)])
        experts.append(trip)
        first = first or trip
    shared = tuple(organ(*s)[0] for s in [(inter, hidden), (inter, hidden), (hidden, inter)])
    norm_w = (rng.standard_normal(hidden) * 0.1).astype(np.float32)
    router_w = (rng.standard_normal((n_experts, hidden)) * 0.02).astype(np.float32)
    gate_w = (rng.standard_normal(hidden) * 0.02).astype(np.float32) if shared_gate else None
    layer = oracle.MoeLayer(hidden, inter, n_experts, top_k, norm_w, router_w, experts,
                            shared=shared, shared_gate_w=gate_w)
    return layer, rng, experts, shared, router_w, norm_w, gate_w


@pytest.mark.parametrize("kind", ["q4", "mixed"])
def test_moe_layer_vs_f64_authority(oracle, kind):
    layer, rng, *_ = _small_layer(oracle, kind)
    h = rng.standard_normal(256).astype(np.float32)
    out, ids, w, xn, logits = layer.forward(h)
    assert len(set(ids.tolist())) == 4 and abs(float(w.sum()) - 1) < 1e-4
    ref = layer.forward_f64(h, ids)
    assert oracle.relative_l2(out, ref) < 2e-6
    # the residual is carried: the delta is small relative to h but nonzero
    assert 0 < np.linalg.norm(out - h) < np.linalg.norm(h)


def test_moe_layer_route_is_router_of_normed_input(oracle):
    layer, rng, experts, shared, router_w, norm_w, gate_w = _small_layer(oracle)
    h = rng.standard_normal(256).astype(np.float32)
    out, ids, w, xn, logits = layer.forward(h)
    assert np.array_equal(xn, oracle.rmsnorm_1p(h, norm_w))
    assert np.array_equal(logits, oracle.gemv_f32(router_w, xn))
    ids2, w2 = oracle.router_softmax_topk(logits, 4)
    assert np.array_equal(ids, ids2) and np.array_equal(w, w2)


def test_moe_layer_zero_experts_leaves_gated_shared(oracle):
    layer, rng, experts, shared, router_w, norm_w, gate_w = _small_layer(oracle, zero_experts=True)
    h = rng.standard_normal(256).astype(np.float32)
    out, *_ = layer.forward(h)
    # all routed and shared weights are zero -> every MLP is zero -> out == h exactly
    assert np.array_equal(out, h)


def test_moe_layer_identical_experts_route_invariant(oracle):
    layer, rng, experts, shared, router_w, norm_w, gate_w = _small_layer(oracle, identical=True)
    h = rng.standard_normal(256).astype(np.float32)
    out, ids, w, xn, _ = layer.forward(h)
    # sum_r w_r * f(xn) with sum w_r = 1 -> f(xn) (+ gated shared), whatever the route
    ref = layer.forward_f64(h, ids)
    e = oracle.Organ
    a = np.empty(128, np.float32)
    single = np.empty(256, np.float32)
    import ctypes as C
    lib = oracle.lib()
    t = experts[0]
    lib.hko_mlp(C.byref(t[0].c), C.byref(t[1].c), C.byref(t[2].c), xn.ctypes.data,
                a.ctypes.data, single.ctypes.data)
    sh = np.empty(256, np.float32)
    lib.hko_mlp(C.byref(shared[0].c), C.byref(shared[1].c), C.byref(shared[2].c), xn.ctypes.data,
                None, sh.ctypes.data)
    g = 1 / (1 + np.exp(-np.dot(gate_w.astype(np.float64), xn.astype(np.float64))))
    approx = h.astype(np.float64) + single.astype(np.float64) + g * sh.astype(np.float64)
    assert oracle.relative_l2(out, approx) < 1e-6
    assert oracle.relative_l2(out, ref) < 2e-6
    del e


# ------------------------------------------------------------------ noaux_tc MoE block (routed_moe)

def _small_noaux(oracle, hidden=256, inter=128, n_experts=32, top_k=4, n_group=4, topk_group=2, seed=1,
                 norm=True, scaling=2.5, zero_experts=False, identical=False):
    rng = np.random.default_rng(seed)

    def organ(rows, cols, zero=False):
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        if zero:
            w[:] = 0
        return oracle.Organ.q4(w, 32)

    experts, first = [], None
    for e in range(n_experts):
        if identical and first is not None:
            experts.append(first)
            continue
        trip = tuple(organ(*s, zero=zero_experts) for s in [(inter, hidden), (inter, hidden), (hidden, inter)])
        experts.append(trip)
        first = first or trip
    shared = tuple(organ(*s) for s in [(inter, hidden), (inter, hidden), (hidden, inter)])
    router_w = (rng.standard_normal((n_experts, hidden)) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(n_experts) * 0.01).astype(np.float32)
    m = oracle.NoauxMoe(hidden, n_experts, top_k, n_group, topk_group, norm, scaling, router_w, bias,
                        experts, shared)
    return m, rng, experts, shared, router_w, bias


def _mlp(oracle, trip, x):
    import ctypes as C
    out = np.empty(trip[2].rows, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    rc = oracle.lib().hko_mlp(C.byref(trip[0].c), C.byref(trip[1].c), C.byref(trip[2].c), x.ctypes.data, None,
                              out.ctypes.data)
    assert rc == 0
    return out


@pytest.mark.parametrize("norm,scaling", [(True, 2.5), (False, 1.0)])
def test_noaux_moe_vs_f64_authority(oracle, norm, scaling):
    m, rng, *_ = _small_noaux(oracle, norm=norm, scaling=scaling)
    for _ in range(3):
        x = rng.standard_normal(256).astype(np.float32)
        out, ids, w, logits = m.forward(x)
        assert len(set(ids.tolist())) == 4
        if norm:
            assert abs(float(w.sum()) / scaling - 1) < 1e-5
        assert oracle.relative_l2(out, m.forward_f64(x, ids)) < 2e-6


def test_noaux_moe_route_is_noaux_tc_of_router_logits(oracle):
    m, rng, experts, shared, router_w, bias = _small_noaux(oracle)
    x = rng.standard_normal(256).astype(np.float32)
    out, ids, w, logits = m.forward(x)
    assert np.array_equal(logits, oracle.gemv_f32(router_w, x))
    ids2, w2 = oracle.router_noaux_tc(logits, bias, 4, 2, 4, True, 2.5)
    assert np.array_equal(ids, ids2) and np.array_equal(w, w2)


def test_noaux_moe_combines_in_ascending_expert_order(oracle):
    """routed accumulates o*w over the experts sorted by id, then adds the
    shared output: rebuilt from per-expert MLPs in that order it is bit-exact,
    while the route order gives a different rounding on some input."""
    m, rng, experts, shared, *_ = _small_noaux(oracle)
    differs = False
    for _ in range(8):
        x = rng.standard_normal(256).astype(np.float32)
        out, ids, w, _ = m.forward(x)
        outs = {int(e): _mlp(oracle, experts[int(e)], x) for e in ids}
        asc = np.zeros(256, np.float32)
        for s in sorted(range(4), key=lambda s: int(ids[s])):
            asc += outs[int(ids[s])] * w[s]
        asc += _mlp(oracle, shared, x)
        assert np.array_equal(out, asc)
        route = np.zeros(256, np.float32)
        for s in range(4):
            route += outs[int(ids[s])] * w[s]
        route += _mlp(oracle, shared, x)
        differs |= not np.array_equal(out, route)
    assert differs


def test_noaux_moe_zero_experts_is_shared_only(oracle):
    m, rng, experts, shared, *_ = _small_noaux(oracle, zero_experts=True)
    x = rng.standard_normal(256).astype(np.float32)
    out, *_ = m.forward(x)
    # every routed MLP is exactly zero: routed = 0, out = 0 + mlp_shared(x) exactly
    sh = _mlp(oracle, shared, x)
    assert np.any(sh != 0) and np.array_equal(out, sh)


def test_noaux_moe_identical_experts_scale_by_routed_factor(oracle):
    m, rng, experts, shared, *_ = _small_noaux(oracle, identical=True, norm=True, scaling=2.5)
    x = rng.standard_normal(256).astype(np.float32)
    out, ids, w, _ = m.forward(x)
    f = _mlp(oracle, experts[0], x).astype(np.float64)
    sh = _mlp(oracle, shared, x).astype(np.float64)
    # sum_r w_r f(x) with sum_r w_r = 2.5 (renormalised, then scaled) -> 2.5 f(x) + shared
    assert oracle.relative_l2(out, 2.5 * f + sh) < 1e-6
