"""The oracle's moe_suffix over the mixed-1p5-v1 organ kinds (q8 HGRAVU01,
binary HGRAVB01, HGRAVR02 binary + Rice residual, HGRAVS01 low-rank).

Pins the organ dispatch of the oracle's layer: each kind's organ matvec is
bit-identical to its standalone codec routine (those are pinned by their own
known-answer tests), and the layer's FP64 path equals a numpy FP64
composition over the densely decoded weights (decoders independent of the
matvec code), so a wrong operand, a swapped gate/up, a missing residual or a
transposed factor fails here."""
import numpy as np
import pytest

from tests import hk_testutil as U


def _key(oracle, *idx):
    v = 0x515
    for i in idx:
        v = (v << 10) + i
    return oracle.stream_key(U.SEED, v)


def _rice_dense(oracle, p):
    d = oracle.bin_decode(p.bin_scales, p.bin_signs, p.rows, p.cols).reshape(-1).astype(np.float64)
    s = oracle.f16_to_f32(p.res_scale)
    bits = np.unpackbits(p.res_signs, bitorder="little")[:p.count]
    np.add.at(d, p.indices.astype(np.int64), np.where(bits == 1, s, -s))
    return d.reshape(p.rows, p.cols)


def test_mixed_organ_kinds_match_codec_routines(oracle):
    rows, cols, rank = 64, 256, 32
    w = oracle.normal(_key(oracle, 1), rows * cols, 0.05).reshape(rows, cols)
    x = oracle.normal(_key(oracle, 2), cols, 1.0)
    o8 = oracle.Organ.uniform8(w)
    assert np.array_equal(o8.matvec(x), oracle.uniform_matvec(o8.scales, o8.codes, rows, cols, x, 8, 64))
    orc = oracle.Organ.rice_q1(w, 0.03)
    assert np.array_equal(orc.matvec(x), oracle.rice_q1_matvec(orc.rice, x))
    lw = oracle.normal(_key(oracle, 3), rows * rank, 0.05).reshape(rows, rank)
    rw = oracle.normal(_key(oracle, 4), rank * cols, 0.05).reshape(rank, cols)
    olr = oracle.Organ.low_rank(lw, rw)
    want = oracle.hgravs01_matvec((olr.scales, olr.codes), olr.right, rows, rank, cols, x, 3, 64)
    assert np.array_equal(olr.matvec(x), want)


def _silu(g):
    return g / (1.0 + np.exp(-g))


@pytest.mark.parametrize("shared", [True, False])
def test_mixed_layer_f64_matches_dense_composition(oracle, shared):
    H, I, SI, E, K, rank = 256, 128, 128, 16, 4, 32
    nw = oracle.normal(_key(oracle, 10), H, 0.02)
    o_r = oracle.Organ.uniform8(oracle.normal(_key(oracle, 11), E * H, 0.05).reshape(E, H))
    R = oracle.uniform_decode(o_r.scales, o_r.codes, E, H, 8, 64).reshape(E, H)
    experts, dense = [], []
    for e in range(E):
        g = oracle.Organ.binary(oracle.normal(_key(oracle, 12, e), I * H, 0.05).reshape(I, H))
        u = oracle.Organ.rice_q1(oracle.normal(_key(oracle, 13, e), I * H, 0.05).reshape(I, H), 0.02)
        d = oracle.Organ.low_rank(oracle.normal(_key(oracle, 14, e), H * rank, 0.05).reshape(H, rank),
                                  oracle.normal(_key(oracle, 15, e), rank * I, 0.05).reshape(rank, I))
        experts.append((g, u, d))
        dense.append((oracle.bin_decode(g.scales, g.codes, I, H).reshape(I, H).astype(np.float64),
                       _rice_dense(oracle, u.rice),
                       oracle.uniform_decode(d.scales, d.codes, H, rank, 3, 64).reshape(H, rank).astype(np.float64),
                       oracle.uniform_decode(d.right[0], d.right[1], rank, I, 3, 64).reshape(rank, I)
                       .astype(np.float64)))
    sh = sg = None
    if shared:
        ws = [oracle.normal(_key(oracle, 16, j), SI * H, 0.05).reshape(SI, H) for j in range(2)]
        ws.append(oracle.normal(_key(oracle, 16, 2), H * SI, 0.05).reshape(H, SI))
        sh = tuple(oracle.Organ.uniform8(w) for w in ws)
        og = oracle.Organ.uniform8(oracle.normal(_key(oracle, 17), H, 0.05).reshape(1, H))
        sg = oracle.uniform_decode(og.scales, og.codes, 1, H, 8, 64).reshape(H)
    L = oracle.MoeLayer(H, I, E, K, nw, R, experts, shared=sh, shared_gate_w=sg)
    h = oracle.normal(_key(oracle, 18), H, 1.0)
    out, ids, wts, xn, logits = L.forward(h)
    # f32 pieces the oracle reports
    assert np.array_equal(xn, oracle.rmsnorm_1p(h, nw))
    rid, rw = oracle.router_softmax_topk(logits, K)
    assert ids.tolist() == list(rid) and np.array_equal(wts, rw)
    # FP64 composition on the dense weights, at the same ids and weights
    h64 = h.astype(np.float64)
    x64 = h64 / np.sqrt(np.mean(h64 * h64) + 1e-6) * (1.0 + nw.astype(np.float64))
    l64 = R.astype(np.float64) @ x64
    p = np.exp(l64 - l64.max())
    p /= p.sum()
    w64 = p[ids] / p[ids].sum()
    acc = np.zeros(H)
    for r, e in enumerate(ids):
        G, U_, Ld, Rd = dense[e]
        acc += w64[r] * (Ld @ (Rd @ (_silu(G @ x64) * (U_ @ x64))))
    if shared:
        S = [oracle.uniform_decode(o.scales, o.codes, o.rows, o.cols, 8, 64).reshape(o.rows, o.cols)
             .astype(np.float64) for o in sh]
        gate = 1.0 / (1.0 + np.exp(-(sg.astype(np.float64) @ x64)))
        acc += gate * (S[2] @ (_silu(S[0] @ x64) * (S[1] @ x64)))
    want = h64 + acc
    got64 = L.forward_f64(h, ids)
    assert np.max(np.abs(got64 - want)) <= 1e-9 * np.max(np.abs(want))
    assert oracle.relative_l2(out, want) < 2e-5
