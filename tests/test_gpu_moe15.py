"""GPU parity of the mixed-1p5-v1 MoE layer (hk_moe15_decode_layer) against
the oracle's moe_suffix over the same packed organs: routed gate HGRAVB01,
up HGRAVR02 (binary + Rice residual), down HGRAVS01 (3-bit G64 factors);
router, shared-expert gate and shared expert HGRAVU01 q8 (the oracle gets
the router and shared gate as their decoded q8 weights, which is
uniform_factor_matvec_f32's arithmetic).

Router ids must match exactly under the margin rule; weights within 1e-5
relative (the q8 router runs on the fixed-point engine, so its logits agree
with the serial f32 dot to about 1e-7 relative and a peaked softmax carries
that into its largest weight); layer outputs within 2e-5 rel-L2 of the
oracle's f32 moe_suffix and of the FP64 authority on the GPU's ids."""
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


def _key(oracle, tag, *idx):
    v = tag
    for i in idx:
        v = (v << 12) + i
    return oracle.stream_key(U.SEED, v)


def _q8(ctx, oracle, w):
    from hawking_amd.organs import UniformFactorPacked
    o = oracle.Organ.uniform8(w)
    return UniformFactorPacked(ctx, o.scales, o.codes, o.rows, o.cols), o


def build_layer(ctx, oracle, H, I, SI, E, K, rank, tag=0x15, ratio=0.02):
    """Random weights packed by the oracle's packers, bound on the device
    (Mixed15Layer) and wrapped for the oracle (MoeLayer)."""
    from hawking_amd.moe import Mixed15Layer
    from hawking_amd.organs import BinaryGroupPacked, HgravS01LowRank, RiceQ1Packed, UniformFactor3
    nw = oracle.normal(_key(oracle, tag, 1), H, 0.02)
    router_w = oracle.normal(_key(oracle, tag, 2), E * H, 0.05).reshape(E, H)
    router, ro = _q8(ctx, oracle, router_w)
    router_dec = oracle.uniform_decode(ro.scales, ro.codes, E, H, 8, 64).reshape(E, H)
    oexp, gexp = [], []
    for e in range(E):
        gw = oracle.normal(_key(oracle, tag, 3, e), I * H, 0.05).reshape(I, H)
        uw = oracle.normal(_key(oracle, tag, 4, e), I * H, 0.05).reshape(I, H)
        lw = oracle.normal(_key(oracle, tag, 5, e), H * rank, 0.05).reshape(H, rank)
        rw = oracle.normal(_key(oracle, tag, 6, e), rank * I, 0.05).reshape(rank, I)
        og = oracle.Organ.binary(gw)
        ou = oracle.Organ.rice_q1(uw, ratio)
        od = oracle.Organ.low_rank(lw, rw)
        p = ou.rice
        g = BinaryGroupPacked(ctx, og.scales, og.codes, I, H)
        u = RiceQ1Packed(ctx, p.rows, p.cols, p.bin_scales, p.bin_signs, p.first, p.rice_k, p.rice, p.count,
                         p.res_scale, p.res_signs)
        d = HgravS01LowRank(UniformFactor3(ctx, od.scales, od.codes, H, rank),
                            UniformFactor3(ctx, od.right[0], od.right[1], rank, I))
        oexp.append((og, ou, od))
        gexp.append((g, u, d))
    shared = oshared = sgate = sgate_dec = None
    if SI:
        sg_w = oracle.normal(_key(oracle, tag, 7), H, 0.05).reshape(1, H)
        sgate, so = _q8(ctx, oracle, sg_w)
        sgate_dec = oracle.uniform_decode(so.scales, so.codes, 1, H, 8, 64).reshape(H)
        ws = [oracle.normal(_key(oracle, tag, 8, j), SI * H, 0.05).reshape(SI, H) for j in range(2)]
        ws.append(oracle.normal(_key(oracle, tag, 8, 2), H * SI, 0.05).reshape(H, SI))
        pairs = [_q8(ctx, oracle, w) for w in ws]
        shared = tuple(p[0] for p in pairs)
        oshared = tuple(p[1] for p in pairs)
    layer = Mixed15Layer(ctx, nw, router, gexp, K, shared=shared, shared_gate=sgate)
    ref = oracle.MoeLayer(H, I, E, K, nw, router_dec, oexp, shared=oshared, shared_gate_w=sgate_dec)
    return layer, ref


def router_weights_f64(ref, h, ids, eps=1e-6):
    """The routed weights in FP64 (RMSNorm(1+w), the decoded q8 router, softmax,
    renormalised over the selection): the numeric authority for the weights."""
    h64 = np.asarray(h, np.float64)
    xn = h64 / np.sqrt(np.dot(h64, h64) / h64.size + eps) * (1.0 + ref.norm_w.astype(np.float64))
    lg = ref.router_w.astype(np.float64) @ xn
    p = np.exp(lg - lg.max())
    sel = p[np.asarray(ids)] / p.sum()
    return sel / sel.sum()


def _check(ctx, oracle, layer, ref, h, K):
    out, ids, w = layer.moe_suffix(h)
    assert ctx.device_status() == 0
    rout, rids, rw, _, logits = ref.forward(h)
    if U.router_margin_ok(logits, K):
        assert ids.tolist() == rids.tolist()
        # the weights within 1e-6 of the FP64 authority; the serial f32 oracle
        # (whose own router dot differs from FP64 by up to ~1e-6) within 2e-6
        w64 = router_weights_f64(ref, h, ids)
        print("[gpu-case] router weight max abs dev: vs FP64", float(np.max(np.abs(w - w64))),
              "oracle vs FP64", float(np.max(np.abs(rw - w64))), "vs oracle", float(np.max(np.abs(w - rw))), flush=True)
        assert np.all(np.abs(w - w64) <= 1e-6)
        assert np.all(np.abs(w - rw) <= 2e-6)
        assert oracle.relative_l2(out, rout) < TOL
    assert oracle.relative_l2(out, ref.forward_f64(h, ids)) < TOL
    return ids


@pytest.mark.parametrize("H,I,SI,E,K,rank", [
    (512, 256, 256, 32, 4, 64),     # one-lane router rows (E <= 64)
    (768, 128, 0, 128, 10, 32),     # no shared expert, E <= 256 form
    (512, 128, 128, 320, 8, 96),    # E > 256 form of the selection
    (2048, 512, 512, 64, 10, 160),  # the artifact's Qwen3-Next shapes (r160 down), 64 experts
    (1024, 256, 256, 48, 16, 64),   # the largest top_k (one wave per slot in the down-left block)
    (512, 224, 128, 37, 6, 64),     # n_experts not a multiple of 4 (padded tile-start rows), a partial router tile
    (512, 128, 128, 512, 10, 32),   # the largest n_experts the layer admits (the artifact's 512)
])
def test_mixed15_layer_matches_oracle(ctx, oracle, H, I, SI, E, K, rank):
    say("mixed15 layer", H, I, SI, E, K, rank)
    layer, ref = build_layer(ctx, oracle, H, I, SI, E, K, rank)
    ctx.device_status()
    seen = set()
    for t in range(4):
        h = oracle.normal(_key(oracle, 0x16, t, E), H, 1.0)
        seen.update(_check(ctx, oracle, layer, ref, h, K).tolist())
    assert len(seen) > K  # the routes differ between inputs
    layer.free()


def test_mixed15_layer_is_repeatable_and_chains(ctx, oracle):
    """Three layers chained on the device (h_{l+1} = layer_l(h_l)) vs the
    oracle layer by layer; a second pass gives the same bits."""
    H, I, SI, E, K, rank = 512, 128, 128, 64, 6, 32
    say("mixed15 chain")
    layers = [build_layer(ctx, oracle, H, I, SI, E, K, rank, tag=0x20 + l) for l in range(3)]
    h0 = oracle.normal(_key(oracle, 0x17, 0), H, 1.0)
    bufs = [ctx.to_device(h0)] + [ctx.empty(H) for _ in layers]
    ids = ctx.empty(len(layers) * K, np.int32)
    for rep in range(2):
        for l, (layer, _) in enumerate(layers):
            layer.decode_device(bufs[l], bufs[l + 1], ids.offset(K * l))
        outs = [b.download() for b in bufs[1:]]
        if rep == 0:
            first = outs
        else:
            for a, b in zip(first, outs):
                assert np.array_equal(a, b)
    assert ctx.device_status() == 0
    got_ids = ids.download().reshape(len(layers), K)
    h = h0
    for l, (layer, ref) in enumerate(layers):
        rout, rids, _, _, logits = ref.forward(h)
        if U.router_margin_ok(logits, K):
            assert got_ids[l].tolist() == rids.tolist()
        assert oracle.relative_l2(first[l], ref.forward_f64(h, got_ids[l])) < TOL
        h = first[l]
    for layer, _ in layers:
        layer.free()


def test_mixed15_layer_flags_nonfinite_hidden_state(ctx, oracle):
    """A NaN in h is latched in the device status word; every kernel still
    ends normally and the next clean call matches the oracle."""
    H, I, SI, E, K, rank = 512, 128, 128, 32, 4, 32
    say("mixed15 non-finite")
    layer, ref = build_layer(ctx, oracle, H, I, SI, E, K, rank, tag=0x30)
    ctx.device_status()
    h = np.ones(H, np.float32)
    h[5] = np.nan
    layer.moe_suffix(h)
    assert ctx.device_status() != 0
    _check(ctx, oracle, layer, ref, oracle.normal(_key(oracle, 0x31, 0), H, 1.0), K)
    layer.free()


def test_mixed15_layer_rejects_bad_geometry(ctx, oracle):
    from hawking_amd._lib import HK_E_GEOMETRY, HK_E_UNSUPPORTED, HawkingError
    from hawking_amd.moe import Mixed15Layer
    H, I, SI, E, K, rank = 512, 128, 0, 8, 2, 32
    say("mixed15 rejections")
    layer, _ = build_layer(ctx, oracle, H, I, SI, E, K, rank, tag=0x40)
    router, experts = layer._keep[0], layer._keep[1]
    nw = np.zeros(H, np.float32)
    with pytest.raises(HawkingError) as e:
        Mixed15Layer(ctx, nw, router, experts, E + 1)
    assert e.value.code == HK_E_UNSUPPORTED
    swapped = [(t[1], t[0], t[2]) for t in experts]  # an up without a residual as the gate
    with pytest.raises(HawkingError) as e:
        Mixed15Layer(ctx, nw, router, swapped, K)
    assert e.value.code == HK_E_GEOMETRY
    with pytest.raises(HawkingError) as e:
        Mixed15Layer(ctx, nw, router, experts[:E - 1], K)  # router rows != n_experts
    assert e.value.code == HK_E_GEOMETRY
    layer.free()
