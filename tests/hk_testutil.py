"""Shared helpers for the parity tests: the synthetic model definition seen
from the oracle side.

The product generates weights on the device from (seed, stream id); these
helpers regenerate any single tensor on the host with the oracle's copy of
the generator so that the CPU oracle runs on bit-identical inputs.
Stream ids: ((layer+1) << 40) | (expert << 8) | proj, proj 0/1/2 =
gate/up/down, 16 = RMSNorm weight, 17 = router, 18 = shared-expert gate,
19 = router bias (noaux_tc), 32+p = mixed-format coins of projection p;
expert n_experts = shared expert.
"""
from __future__ import annotations

import numpy as np

SEED = 0x48415752  # "HAWR"
SIGMA_W = 0.02
SIGMA_NORM = 0.02
SIGMA_BIAS = 0.01
PROJ_NORM, PROJ_ROUTER, PROJ_SHARED_GATE, PROJ_BIAS, PROJ_COIN = 16, 17, 18, 19, 32
HK_Q4, HK_BIN, HK_MIXED, HK_F32 = 0, 1, 2, 3


def stream_id(layer: int, expert: int, proj: int) -> int:
    return ((layer + 1) << 40) | (expert << 8) | proj


def organ_shape(shape, expert: int, proj: int):
    inter = shape.shared_inter if expert == shape.n_experts else shape.inter
    return (inter, shape.hidden) if proj < 2 else (shape.hidden, inter)


def weights(oracle, seed, layer, expert, proj, rows, cols, sigma=SIGMA_W):
    key = oracle.stream_key(seed, stream_id(layer, expert, proj))
    return oracle.normal(key, rows * cols, sigma).reshape(rows, cols)


def coins(oracle, seed, layer, expert, proj, groups):
    return oracle.mixed_coins(oracle.stream_key(seed, stream_id(layer, expert, PROJ_COIN + proj)), groups)


def oracle_organ(oracle, seed, shape, layer, expert, proj):
    rows, cols = organ_shape(shape, expert, proj)
    w = weights(oracle, seed, layer, expert, proj, rows, cols)
    if shape.expert_kind == HK_Q4:
        return oracle.Organ.q4(w, shape.expert_group)
    sel = coins(oracle, seed, layer, expert, proj, rows * cols // 128)
    return oracle.Organ.mixed_from(w, sel)


def dense(oracle, seed, shape, layer):
    H, E = shape.hidden, shape.n_experts
    norm = oracle.normal(oracle.stream_key(seed, stream_id(layer, 0, PROJ_NORM)), H, SIGMA_NORM)
    router = oracle.normal(oracle.stream_key(seed, stream_id(layer, 0, PROJ_ROUTER)), E * H, SIGMA_W).reshape(E, H)
    gate = oracle.normal(oracle.stream_key(seed, stream_id(layer, 0, PROJ_SHARED_GATE)), H, SIGMA_W)
    return norm, router, gate


def oracle_layer(oracle, seed, shape, layer, h):
    """Oracle moe_suffix for one synthetic layer, generating only the routed
    experts (plus the shared one).  Returns (layer_obj, out, ids, weights)."""
    norm, router, gate = dense(oracle, seed, shape, layer)
    xn = oracle.rmsnorm_1p(h, norm, shape.eps)
    logits = oracle.gemv_f32(router, xn)
    ids, _ = oracle.router_softmax_topk(logits, shape.top_k, getattr(shape, "route_tie_eps", 0.0))
    experts = [None] * shape.n_experts
    for e in ids.tolist():
        experts[e] = tuple(oracle_organ(oracle, seed, shape, layer, e, p) for p in range(3))
    shared = None
    if shape.shared_inter:
        shared = tuple(oracle_organ(oracle, seed, shape, layer, shape.n_experts, p) for p in range(3))
    L = oracle.MoeLayer(shape.hidden, shape.inter, shape.n_experts, shape.top_k, norm, router, experts,
                        shared=shared, shared_gate_w=gate if (shape.shared_gate and shape.shared_inter) else None,
                        eps=shape.eps, tie_eps=getattr(shape, "route_tie_eps", 0.0))
    out, ids2, w, xn2, logits2 = L.forward(h)
    assert np.array_equal(ids, ids2)
    return L, out, ids2, w, logits2


def oracle_layer_cached(oracle, seed, shape, layer, h, cache, pool=None):
    """oracle_layer with the generated expert organs kept in `cache`
    ((layer, expert) -> (gate, up, down)) and generated on `pool` (a
    thread pool: the oracle's C calls release the GIL).  Returns
    (layer_obj, out, ids, weights, logits, xn)."""
    norm, router, gate = cache.get(("dense", layer)) or dense(oracle, seed, shape, layer)
    cache[("dense", layer)] = (norm, router, gate)
    xn = oracle.rmsnorm_1p(h, norm, shape.eps)
    logits = oracle.gemv_f32(router, xn)
    ids, _ = oracle.router_softmax_topk(logits, shape.top_k, getattr(shape, "route_tie_eps", 0.0))
    want = [int(e) for e in ids] + ([shape.n_experts] if shape.shared_inter else [])
    todo = [(e, p) for e in want if (layer, e) not in cache for p in range(3)]
    make = lambda ep: oracle_organ(oracle, seed, shape, layer, ep[0], ep[1])
    made = list(pool.map(make, todo)) if pool is not None else [make(t) for t in todo]
    for i in range(0, len(todo), 3):
        cache[(layer, todo[i][0])] = tuple(made[i:i + 3])
    experts = [None] * shape.n_experts
    for e in ids.tolist():
        experts[e] = cache[(layer, e)]
    shared = cache[(layer, shape.n_experts)] if shape.shared_inter else None
    L = oracle.MoeLayer(shape.hidden, shape.inter, shape.n_experts, shape.top_k, norm, router, experts,
                        shared=shared, shared_gate_w=gate if (shape.shared_gate and shape.shared_inter) else None,
                        eps=shape.eps, tie_eps=getattr(shape, "route_tie_eps", 0.0))
    out, ids2, w, xn2, logits2 = L.forward(h)
    assert np.array_equal(ids, ids2)
    return L, out, ids2, w, logits2, xn2


def tie_window_margin_ok(logits: np.ndarray, eps: float, margin: float = 1e-8) -> bool:
    """Margin rule for the tie-window router: the selection depends only on
    whether q_i - q_j exceeds eps for pairs of normalised probabilities
    (q = softmax(logits), from the oracle's f32 logits), so every pairwise
    difference must stay at least `margin` away from eps; the device's
    logits differ from the oracle's by about 1e-7 relative, which moves a q
    by far less than that."""
    l = logits.astype(np.float64)
    q = np.exp(l - l.max())
    q /= q.sum()
    d = q[:, None] - q[None, :]
    return float(np.min(np.abs(d - eps))) >= margin


def router_margin_ok(logits: np.ndarray, k: int, rel: float = 1e-4) -> bool:
    """Router margin rule: the f64 gap between the k-th and (k+1)-th
    score must be >= rel * max|score| for ids to be compared bit-exactly."""
    l64 = np.sort(logits.astype(np.float64))[::-1]
    if k >= l64.size:
        return True
    return (l64[k - 1] - l64[k]) >= rel * np.max(np.abs(l64))


def organ_dict(o) -> dict:
    """Canonical organ arrays of an oracle Organ, for MoeModel.set_layer."""
    if o.kind == HK_Q4:
        return {"kind": HK_Q4, "group": o.group, "rows": o.rows, "cols": o.cols, "scales": o.scales, "codes": o.codes}
    m = o.mixed
    return {"kind": HK_MIXED, "rows": o.rows, "cols": o.cols, "tags": m.tags, "bin_scales": m.bin_scales,
            "bin_signs": m.bin_signs, "q2_scales": m.q2_scales, "q2_codes": m.q2_codes}


def router_bias(oracle, seed, shape, layer):
    return oracle.normal(oracle.stream_key(seed, stream_id(layer, 0, PROJ_BIAS)), shape.n_experts, SIGMA_BIAS)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def noaux_margin_ok(logits, bias, n_group, topk_group, k, rel=1e-4) -> bool:
    """Router margin rule for noaux_tc, in f64: the chosen groups and the k-th /
    (k+1)-th candidate must be separated by >= rel * max|value|."""
    s = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    c = s + bias.astype(np.float64)
    per = c.size // n_group
    gs = np.array([np.sort(c[g * per:(g + 1) * per])[::-1][:2].sum() for g in range(n_group)])
    if topk_group < n_group:
        o = np.sort(gs)[::-1]
        if o[topk_group - 1] - o[topk_group] < rel * np.max(np.abs(o)):
            return False
    chosen = np.argsort(-gs, kind="stable")[:topk_group]
    cand = np.sort(np.concatenate([c[g * per:(g + 1) * per] for g in chosen]))[::-1]
    if k < cand.size and cand[k - 1] - cand[k] < rel * np.max(np.abs(cand)):
        return False
    return True


def oracle_noaux(oracle, seed, shape, layer, x):
    """Oracle routed_moe for one synthetic token x (f32), generating only the
    routed experts and the shared one.  Returns (block, out, ids, weights, logits)."""
    _, router, _ = dense(oracle, seed, shape, layer)
    bias = router_bias(oracle, seed, shape, layer)
    logits = oracle.gemv_f32(router, x)
    ids, _ = oracle.router_noaux_tc(logits, bias, shape.n_group, shape.topk_group, shape.top_k,
                                    shape.norm_topk_prob, shape.routed_scaling_factor)
    experts = [None] * shape.n_experts
    for e in ids.tolist():
        experts[e] = tuple(oracle_organ(oracle, seed, shape, layer, e, p) for p in range(3))
    shared = None
    if shape.shared_inter:
        shared = tuple(oracle_organ(oracle, seed, shape, layer, shape.n_experts, p) for p in range(3))
    M = oracle.NoauxMoe(shape.hidden, shape.n_experts, shape.top_k, shape.n_group, shape.topk_group,
                        shape.norm_topk_prob, shape.routed_scaling_factor, router, bias, experts, shared)
    out, ids2, w, logits2 = M.forward(x)
    assert np.array_equal(ids, ids2)
    return M, out, ids2, w, logits2


# ---------------------------------------------------------------- synthetic mixed-1p5-v1 model
def mixed15_weights(oracle, seed, d, layer, expert, proj):
    """The draws of one tensor of hawking_amd.moe.synthetic_mixed15_layers
    (the device's generator stream, regenerated by the oracle)."""
    from hawking_amd.moe import mixed15_stream_id, mixed15_tensor
    kind, rows, cols, group, sigma = mixed15_tensor(d, expert, proj)
    key = oracle.stream_key(seed, mixed15_stream_id(layer, expert, proj))
    return kind, oracle.normal(key, rows * cols, sigma).reshape(rows, cols)


def mixed15_oracle_expert(oracle, seed, d, layer, expert):
    """Routed expert `expert` of a synthetic mixed-1p5 layer as oracle organs:
    (HGRAVB01 gate, HGRAVR02 up at the 2 % ratio, HGRAVS01 down)."""
    from hawking_amd.moe import MIXED15_DOWN_LEFT, MIXED15_DOWN_RIGHT, MIXED15_GATE, MIXED15_UP
    _, gw = mixed15_weights(oracle, seed, d, layer, expert, MIXED15_GATE)
    _, uw = mixed15_weights(oracle, seed, d, layer, expert, MIXED15_UP)
    _, lw = mixed15_weights(oracle, seed, d, layer, expert, MIXED15_DOWN_LEFT)
    _, rw = mixed15_weights(oracle, seed, d, layer, expert, MIXED15_DOWN_RIGHT)
    return oracle.Organ.binary(gw), oracle.Organ.rice_q1(uw, 0.02), oracle.Organ.low_rank(lw, rw)


def mixed15_oracle_dense(oracle, seed, d, layer):
    """(norm weight, decoded q8 router, decoded q8 shared gate row or None,
    shared expert organs or None) of a synthetic mixed-1p5 layer.  The q8
    router and shared gate reach the oracle as their decoded weights, which
    is uniform_factor_matvec_f32's arithmetic."""
    from hawking_amd.moe import (MIXED15_NORM, MIXED15_ROUTER, MIXED15_SHARED_DOWN, MIXED15_SHARED_GATE,
                                 MIXED15_SHARED_GATE_PROJ, MIXED15_SHARED_UP, mixed15_stream_id)
    H, E = d.hidden, d.n_experts
    norm = oracle.normal(oracle.stream_key(seed, mixed15_stream_id(layer, E, MIXED15_NORM)), H, 0.02)
    _, w = mixed15_weights(oracle, seed, d, layer, E, MIXED15_ROUTER)
    ro = oracle.Organ.uniform8(w)
    router = oracle.uniform_decode(ro.scales, ro.codes, E, H, 8, 64).reshape(E, H)
    if not d.shared_inter:
        return norm, router, None, None
    _, w = mixed15_weights(oracle, seed, d, layer, E, MIXED15_SHARED_GATE)
    so = oracle.Organ.uniform8(w)
    sgate = oracle.uniform_decode(so.scales, so.codes, 1, H, 8, 64).reshape(H)
    shared = tuple(oracle.Organ.uniform8(mixed15_weights(oracle, seed, d, layer, E, p)[1])
                   for p in (MIXED15_SHARED_GATE_PROJ, MIXED15_SHARED_UP, MIXED15_SHARED_DOWN))
    return norm, router, sgate, shared


def mixed15_oracle_layer_cached(oracle, seed, d, layer, h, cache, pool=None, tie_eps=0.0):
    """The oracle's moe_suffix of a synthetic mixed-1p5 layer on h, generating
    only the routed experts (kept in `cache`, generated on `pool`).
    Returns (layer_obj, out, ids, weights, logits)."""
    if ("dense", layer) not in cache:
        cache[("dense", layer)] = mixed15_oracle_dense(oracle, seed, d, layer)
    norm, router, sgate, shared = cache[("dense", layer)]
    logits = oracle.gemv_f32(router, oracle.rmsnorm_1p(h, norm, d.eps))
    ids, _ = oracle.router_softmax_topk(logits, d.top_k, tie_eps)
    todo = [int(e) for e in ids if (layer, int(e)) not in cache]
    make = lambda e: mixed15_oracle_expert(oracle, seed, d, layer, e)
    made = list(pool.map(make, todo)) if pool is not None else [make(e) for e in todo]
    for e, t in zip(todo, made):
        cache[(layer, e)] = t
    experts = [None] * d.n_experts
    for e in ids.tolist():
        experts[e] = cache[(layer, e)]
    L = oracle.MoeLayer(d.hidden, d.inter, d.n_experts, d.top_k, norm, router, experts, shared=shared,
                        shared_gate_w=sgate, eps=d.eps, tie_eps=tie_eps)
    out, ids2, w, _, logits2 = L.forward(h)
    assert np.array_equal(ids, ids2)
    return L, out, ids2, w, logits2


def router_weights_f64(L, h, ids, eps=1e-6):
    """The routed weights in FP64 (RMSNorm(1+w), the layer's router, softmax,
    renormalised over the selection): the numeric authority for the weights."""
    h64 = np.asarray(h, np.float64)
    xn = h64 / np.sqrt(np.dot(h64, h64) / h64.size + eps) * (1.0 + L.norm_w.astype(np.float64))
    lg = L.router_w.astype(np.float64) @ xn
    p = np.exp(lg - lg.max())
    sel = p[np.asarray(ids)] / p.sum()
    return sel / sel.sum()
