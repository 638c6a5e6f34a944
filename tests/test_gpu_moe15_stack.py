"""The mixed-1p5-v1 token at the shape the benchmark times: 48 layers of
hidden 2048, 512 experts x inter 512, top-10, shared expert 512, routed gate
HGRAVB01, up HGRAVR02 (2 % Rice residual), down HGRAVS01 rank 160 (3-bit
G64), q8 router / shared gate / shared expert (forward_token's MoE suffixes,
crates/hawking-core/src/model/qwen80_mixed_hybrid_decode.rs:4682-4736, with
moe_suffix :3636-3752 and routed_wave :2192-2386).

The model is generated and packed on the device
(hawking_amd.moe.synthetic_mixed15_layers, the benchmark's builder); the
oracle regenerates the router, the shared expert and the routed experts each
layer selects (its packers are bit-exact with the device's).  Checks:
  * layer by layer on the device's own hidden state: ids exact under the
    margin rule, weights within 1e-6 of the FP64 authority and 2e-6 of the
    serial f32 oracle (whose own router dot is up to ~1e-6 from FP64), the
    layer output within 2e-5 rel-L2 of the oracle's f32 moe_suffix and of
    the FP64 authority;
  * hk_moe15_decode_stack's ids, weights and final state equal the 48
    chained single-layer calls bit for bit;
  * the final state within 2e-5 rel-L2 of the oracle's own 48-layer f32
    chain (its own routes, which must equal the device's) and FP64 chain.
A near tie at any layer advances the input seed and restarts the walk."""
import concurrent.futures as cf
import sys

import numpy as np
import pytest

from tests import hk_testutil as U

pytestmark = pytest.mark.gpu
TOL = 2e-5
N_LAYERS = 48


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    from hawking_amd.runtime import Context
    return Context(0)


def _oracle_dense_decode(oracle, o):
    """Decoded weights of an oracle organ (rows x cols, f32)."""
    if o.kind == 1:
        return oracle.bin_decode(o.scales, o.codes, o.rows, o.cols)
    if o.kind == 3:
        return oracle.uniform_decode(o.scales, o.codes, o.rows, o.cols, 8, 64)
    if o.kind == 5:
        p = o.rice
        d = oracle.bin_decode(p.bin_scales, p.bin_signs, p.rows, p.cols).reshape(-1).copy()
        sc = oracle.f16_to_f32(p.res_scale)
        bits = np.unpackbits(p.res_signs, bitorder="little")[:p.count]
        np.add.at(d, p.indices.astype(np.int64), np.where(bits == 1, sc, -sc).astype(np.float32))
        return d.reshape(p.rows, p.cols)
    raise ValueError(o.kind)


def _same_bits(got, want, what):
    assert np.array_equal(np.asarray(got, np.float32).view(np.uint32),
                          np.asarray(want, np.float32).reshape(np.shape(got)).view(np.uint32)), what


def test_mixed15_synthetic_organs_decode_bit_exact(ctx, oracle):
    """Every organ kind of the timed model, generated and packed on the device,
    decodes bit for bit to the oracle's pack of the same draws: the router,
    shared gate and shared expert (q8), and routed experts' HGRAVB01 gate,
    HGRAVR02 up and HGRAVS01 factors (3-bit)."""
    from hawking_amd.moe import Mixed15Dims, synthetic_mixed15_layers
    d = Mixed15Dims(n_experts=16)
    say("mixed-1p5 synthetic organs vs the oracle")
    layers, _, _ = synthetic_mixed15_layers(ctx, U.SEED, 2, d)
    for l in (0, 1):
        router, experts, shared, sgate = layers[l]._keep
        norm, router_dec, sgate_dec, oshared = U.mixed15_oracle_dense(oracle, U.SEED, d, l)
        _same_bits(router.decode(), router_dec, f"router {l}")
        _same_bits(sgate.decode().reshape(-1), sgate_dec, f"shared gate {l}")
        for j in range(3):
            _same_bits(shared[j].decode(), _oracle_dense_decode(oracle, oshared[j]), f"shared {j} {l}")
        for e in (0, 7, 15):
            og, ou, od = U.mixed15_oracle_expert(oracle, U.SEED, d, l, e)
            g, u, (lf, rf) = experts[e]
            _same_bits(g.decode(), _oracle_dense_decode(oracle, og), f"gate {l} {e}")
            _same_bits(u.decode(), _oracle_dense_decode(oracle, ou), f"up {l} {e}")
            _same_bits(lf.decode(), oracle.uniform_decode(od.scales, od.codes, d.hidden, d.rank, 3, 64),
                       f"down left {l} {e}")
            _same_bits(rf.decode(), oracle.uniform_decode(od.right[0], od.right[1], d.rank, d.inter, 3, 64),
                       f"down right {l} {e}")
        assert np.array_equal(layers[l]._norm, norm)
    for layer in layers:
        layer.free()


def test_mixed15_token_512_experts_48_layers(ctx, oracle):
    from hawking_amd.moe import Mixed15Dims, mixed15_forward_token, synthetic_mixed15_layers
    d = Mixed15Dims()
    say("mixed-1p5 token: 48 layers x 512 experts, device fill")
    layers, _, _ = synthetic_mixed15_layers(ctx, U.SEED, N_LAYERS, d)
    ctx.device_status()
    cache = {}
    with cf.ThreadPoolExecutor(max_workers=8) as pool:
        for attempt in range(4):
            h0 = oracle.normal(oracle.stream_key(U.SEED, 0x15C4 + attempt), d.hidden, 1.0)
            out, sids, sw = mixed15_forward_token(ctx, layers, h0)
            h = h0
            near_tie = None
            for l in range(N_LAYERS):
                g_out, g_ids, g_w = layers[l].moe_suffix(h)
                L, r_out, r_ids, r_w, logits = U.mixed15_oracle_layer_cached(oracle, U.SEED, d, l, h, cache, pool)
                if not U.router_margin_ok(logits, d.top_k):
                    near_tie = l
                    break
                assert g_ids.tolist() == r_ids.tolist(), f"layer {l}"
                w64 = U.router_weights_f64(L, h, g_ids, d.eps)
                assert np.max(np.abs(g_w - w64)) <= 1e-6, f"layer {l}"
                assert np.max(np.abs(g_w - r_w)) <= 2e-6, f"layer {l}"
                assert oracle.relative_l2(g_out, r_out) < TOL, f"layer {l}"
                assert oracle.relative_l2(g_out, L.forward_f64(h, g_ids)) < TOL, f"layer {l}"
                assert g_ids.tolist() == sids[l].tolist() and np.array_equal(g_w.view(np.uint32),
                                                                              sw[l].view(np.uint32)), f"layer {l}"
                if l % 8 == 7:
                    say(f"layer {l} ok (attempt {attempt})")
                h = g_out
            if near_tie is None:
                break
            say(f"near tie at layer {near_tie}: advancing the input seed")
        else:
            pytest.fail("four input seeds all met a router near tie")
        assert np.array_equal(out.view(np.uint32), h.view(np.uint32)), "stack != chained single-layer calls"
        assert ctx.device_status() == 0

        say("final state vs the oracle's f32 chain and FP64 chain")
        r, r64 = h0, h0.astype(np.float64)
        for l in range(N_LAYERS):
            L, r, r_ids, _, _ = U.mixed15_oracle_layer_cached(oracle, U.SEED, d, l, r, cache, pool)
            assert r_ids.tolist() == sids[l].tolist(), f"oracle chain route differs at layer {l}"
            r64 = L.forward_f64(r64, sids[l])
    assert oracle.relative_l2(out, r) < TOL
    assert oracle.relative_l2(out, r64) < TOL
    for layer in layers:
        layer.free()
