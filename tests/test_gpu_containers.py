"""The loader (hk_organ_from_container / hk_organ_from_hq30 / hk_catalog_*):
the reference's container tests ported (q80_mixed_decode.rs:1508-1640:
parse_binary_container_matches_packer, parse_rice_container_expands_indices,
parse_uniform_q8_container_roundtrip), HGRAVS01 and HQ30 payloads, a written
HQ80M15 catalog, and one failing payload per validation rule.  Bound organs
must decode bit-exactly to the oracle's packed bodies."""
import hashlib
import json
import struct
import sys

import numpy as np
import pytest

from tests import hk_containers as W
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


def _rice_dense(oracle, p):
    d = oracle.bin_decode(p.bin_scales, p.bin_signs, p.rows, p.cols).reshape(-1).copy()
    s = oracle.f16_to_f32(p.res_scale)
    bits = np.unpackbits(p.res_signs, bitorder="little")[:p.count]
    np.add.at(d, p.indices.astype(np.int64), np.where(bits == 1, s, -s).astype(np.float32))
    return d.reshape(p.rows, p.cols)


def test_binary_container_matches_packer(ctx, oracle):
    from hawking_amd.containers import organ_from_container
    rows, cols = 4, 256
    w = oracle.deterministic_matrix(rows, cols, 19)
    s, g = oracle.bin_pack(w)
    say("HGRAVB01", rows, cols)
    o = organ_from_container(ctx, 0, W.binary(s, g, rows, cols))
    assert (o.rows, o.cols) == (rows, cols)
    assert np.array_equal(o.decode(), oracle.bin_decode(s, g, rows, cols))
    x = oracle.deterministic_input(cols)
    assert oracle.relative_l2(o.matvec(x), oracle.bin_matvec(s, g, rows, cols, x)) < TOL


def test_rice_container_expands_indices(ctx, oracle):
    from hawking_amd.containers import organ_from_container
    rows, cols = 8, 128
    p = oracle.rice_q1_pack(oracle.deterministic_matrix(rows, cols, 23), rows, cols, 0.02)
    say("HGRAVR02", rows, cols)
    o = organ_from_container(ctx, 1, W.residual(p))
    assert np.array_equal(o.decode(), _rice_dense(oracle, p))
    x = oracle.deterministic_input(cols)
    assert oracle.relative_l2(o.matvec(x), oracle.rice_q1_matvec(p, x)) < TOL
    y0 = oracle.bin_matvec(p.bin_scales, p.bin_signs, rows, cols, x)
    yd = ctx.to_device(y0)
    o.apply_residual_device(ctx.to_device(x), yd)
    assert np.array_equal(yd.download(), oracle.rice_q1_apply(p, x, y0))


def test_uniform_q8_container_roundtrip(ctx, oracle):
    from hawking_amd.containers import organ_from_container
    rows, cols = 3, 64
    w = oracle.deterministic_matrix(rows, cols, 29)
    s, c = oracle.uniform_pack(w, rows, cols, 8, 64)
    say("HGRAVU01", rows, cols)
    o = organ_from_container(ctx, 3, W.uniform8(s, c, rows, cols))
    assert np.array_equal(o.decode(), oracle.uniform_decode(s, c, rows, cols, 8, 64))


def test_hgravs01_container_two_stage(ctx, oracle):
    from hawking_amd.containers import organ_from_container
    rows, rank, cols = 96, 32, 256
    L = oracle.deterministic_matrix(rows, rank, 3)
    R = oracle.deterministic_matrix(rank, cols, 5)
    left, right = oracle.uniform_pack(L, rows, rank, 3, 64), oracle.uniform_pack(R, rank, cols, 3, 64)
    say("HGRAVS01", rows, rank, cols)
    lr = organ_from_container(ctx, 2, W.hgravs01(left, right, rows, rank, cols))
    assert np.array_equal(lr.left.decode(), oracle.uniform_decode(*left, rows, rank, 3, 64))
    assert np.array_equal(lr.right.decode(), oracle.uniform_decode(*right, rank, cols, 3, 64))
    x = oracle.deterministic_input(cols)
    y = lr.matvec(x)
    assert oracle.relative_l2(y, oracle.hgravs01_matvec(left, right, rows, rank, cols, x, 3, 64)) < TOL


@pytest.mark.parametrize("group", [64, 128])
def test_hq30_uniform_q4_payload(ctx, oracle, group):
    from hawking_amd.containers import organ_from_hq30
    rows, cols = 48, 512
    w = oracle.normal(oracle.stream_key(U.SEED, 0x3A + group), rows * cols, 0.02).reshape(rows, cols)
    s, c = oracle.q4_pack(w, group)
    say("HQ30UQ4", group)
    o = organ_from_hq30(ctx, W.hq30(b"HQ30UQ4\0", group, [rows, cols], s, c))
    assert np.array_equal(o.decode(), oracle.q4_decode(s, c, rows, cols, group))


def test_hq30_binary_payload(ctx, oracle):
    from hawking_amd.containers import organ_from_hq30
    rows, cols = 16, 384
    w = oracle.normal(oracle.stream_key(U.SEED, 0x3B), rows * cols, 0.02).reshape(rows, cols)
    s, g = oracle.bin_pack(w)
    say("HQ30G1B1")
    o = organ_from_hq30(ctx, W.hq30(b"HQ30G1B1", 128, [rows, cols], s, g))
    assert np.array_equal(o.decode(), oracle.bin_decode(s, g, rows, cols))


def _codes():
    from hawking_amd._lib import HK_E_GEOMETRY, HK_E_INVALID_ARG, HK_E_NONFINITE, HK_E_UNSUPPORTED
    return HK_E_INVALID_ARG, HK_E_GEOMETRY, HK_E_UNSUPPORTED, HK_E_NONFINITE


def test_container_validation_rules(ctx, oracle):
    from hawking_amd._lib import HawkingError
    from hawking_amd.containers import organ_from_container, organ_from_hq30
    INV, GEO, UNS, NONF = _codes()
    rows, cols = 4, 256
    s, g = oracle.bin_pack(oracle.deterministic_matrix(rows, cols, 19))
    good = W.binary(s, g, rows, cols)
    p = oracle.rice_q1_pack(oracle.deterministic_matrix(8, 128, 23), 8, 128, 0.02)
    us, uc = oracle.uniform_pack(oracle.deterministic_matrix(3, 64, 29), 3, 64, 8, 64)
    L3 = oracle.uniform_pack(oracle.deterministic_matrix(64, 32, 3), 64, 32, 3, 64)
    R3 = oracle.uniform_pack(oracle.deterministic_matrix(32, 128, 5), 32, 128, 3, 64)
    L4 = oracle.uniform_pack(oracle.deterministic_matrix(64, 32, 3), 64, 32, 4, 64)
    R4 = oracle.uniform_pack(oracle.deterministic_matrix(32, 128, 5), 32, 128, 4, 64)
    hdr_len = struct.unpack_from("<I", good, 8)[0]
    cases = [
        ("magic", 0, b"HGRAVX01" + good[8:], INV),
        ("header past payload", 0, good[:8] + struct.pack("<I", len(good)) + good[12:], GEO),
        ("not JSON", 0, W.wrap(b"HGRAVB01", {}, b"")[:12] + b"{oops" + good[12 + hdr_len:], INV),
        ("root not object", 0, b"HGRAVB01" + struct.pack("<I", 2) + b"[]", INV),
        ("schema", 0, W.binary(s, g, rows, cols, schema="hawking.gravity.other.v1"), INV),
        ("float integer", 0, W.binary(s, g, rows, cols, groups=float(s.size)), INV),
        ("negative", 0, W.binary(s, g, rows, cols, elements=-1), GEO),
        ("group ledger", 0, W.binary(s, g, rows, cols, groups=int(s.size) + 1), GEO),
        ("sign ledger", 0, W.binary(s, g, rows, cols, sign_bytes=int(g.size) - 1), GEO),
        ("body length", 0, good[:-1], GEO),
        ("shape vs elements", 0, W.binary(s, g, rows, cols, shape=[rows, cols + 1]), GEO),
        ("cols % group", 0, W.binary(s, g, rows, cols, shape=[rows * 4, cols // 4]), GEO),
        ("rice value_bits", 1, W.residual(p, value_bits=2), INV),
        ("rice index ledger", 1, W.residual(p, index_bytes=5 + int(p.rice.size)), GEO),
        ("rice first_index_bytes", 1, W.residual(p, first_index_bytes=8), GEO),
        ("rice scale bytes", 1, W.residual(p, residual_scale_bytes=4), GEO),
        ("rice value_scale", 1, W.residual(p, value_scale="max"), INV),
        ("q8 bits", 3, W.uniform8(us, uc, 3, 64, bits=4), GEO),
        ("q8 group", 3, W.uniform8(us, uc, 3, 64, group_size=32), GEO),
        ("s01 fit kind", 2, W.hgravs01(L3, R3, 64, 32, 128, activation_capture={"fit_kind": "weight_space"}), INV),
        ("s01 rank", 2, W.hgravs01(L3, R3, 64, 32, 128, rank=16), GEO),
        ("s01 body", 2, W.hgravs01(L3, R3, 64, 32, 128, left_body_bytes=10), GEO),
        ("s01 4-bit factors", 2, W.hgravs01(L4, R4, 64, 32, 128, bits=4), UNS),
        ("unknown codec", 7, good, INV),
    ]
    for name, codec, payload, code in cases:
        say("reject", name)
        with pytest.raises(HawkingError) as e:
            organ_from_container(ctx, codec, payload)
        assert e.value.code == code, (name, e.value)
    # a Rice stream cut short (ledger consistent) is found when the bind expands it
    q = oracle.rice_q1_pack(oracle.deterministic_matrix(8, 128, 23), 8, 128, 0.02)
    q.rice = q.rice[:max(q.rice.size // 2, 1)]
    with pytest.raises(HawkingError) as e:
        organ_from_container(ctx, 1, W.residual(q))
    assert e.value.code == GEO
    hs, hc = oracle.q4_pack(oracle.deterministic_matrix(4, 128, 7), 64)
    hq_cases = [
        ("hq30 version", W.hq30(b"HQ30UQ4\0", 64, [4, 128], hs, hc, version=2), INV),
        ("hq30 group", W.hq30(b"HQ30UQ4\0", 32, [4, 128], hs, hc), INV),
        ("hq30 reserved", W.hq30(b"HQ30UQ4\0", 64, [4, 128], hs, hc, reserved=1), INV),
        ("hq30 size", W.hq30(b"HQ30UQ4\0", 64, [4, 128], hs, hc)[:-1], GEO),
        ("hq30 rank 3", W.hq30(b"HQ30UQ4\0", 64, [2, 2, 128], hs, hc), GEO),
        ("hq30 magic", b"HQ30XXXX" + W.hq30(b"HQ30UQ4\0", 64, [4, 128], hs, hc)[8:], INV),
    ]
    bad_scale = hs.copy()
    bad_scale[1] = 0x7C00
    hq_cases.append(("hq30 scale", W.hq30(b"HQ30UQ4\0", 64, [4, 128], bad_scale, hc), NONF))
    for name, payload, code in hq_cases:
        say("reject", name)
        with pytest.raises(HawkingError) as e:
            organ_from_hq30(ctx, payload)
        assert e.value.code == code, (name, e.value)


def _catalog_tensors(oracle):
    rb, cb = 64, 256
    bs, bg = oracle.bin_pack(oracle.deterministic_matrix(rb, cb, 19))
    p = oracle.rice_q1_pack(oracle.deterministic_matrix(32, 256, 23), 32, 256, 0.02)
    us, uc = oracle.uniform_pack(oracle.deterministic_matrix(40, 128, 29), 40, 128, 8, 64)
    L = oracle.uniform_pack(oracle.deterministic_matrix(96, 32, 3), 96, 32, 3, 64)
    R = oracle.uniform_pack(oracle.deterministic_matrix(32, 256, 5), 32, 256, 3, 64)
    tensors = [
        ("model.layers.0.mlp.experts.0.gate_proj.weight", 0, 1, [rb, cb], W.binary(bs, bg, rb, cb)),
        ("model.layers.0.mlp.experts.0.up_proj.weight", 1, 2, [32, 256], W.residual(p)),
        ("model.layers.0.mlp.experts.0.down_proj.weight", 2, 3, [96, 256], W.hgravs01(L, R, 96, 32, 256)),
        ("lm_head.weight", 3, 4, [40, 128], W.uniform8(us, uc, 40, 128)),
    ]
    refs = {"gate": (bs, bg), "up": p, "down": (L, R), "lm": (us, uc)}
    return tensors, refs


def test_catalog_open_records_and_load(ctx, oracle, tmp_path):
    from hawking_amd.containers import MixedCatalog
    tensors, refs = _catalog_tensors(oracle)
    mpath = W.write_catalog(tmp_path, tensors)
    say("catalog", len(tensors))
    cat = MixedCatalog(ctx, str(mpath))
    assert (cat.tensor_count, cat.segment_count) == (4, 2)
    assert cat.complete_physical_bpw == 1.4921875
    recs = {r["name"]: r for r in cat.records()}
    for name, codec, organ, shape, payload in tensors:
        r = recs[name]
        assert (r["codec"], r["organ"], r["shape"], r["nbytes"]) == (codec, organ, shape, len(payload))
        assert r["sha256"] == hashlib.sha256(payload).hexdigest()
        assert cat.payload(name) == payload
    gate = cat.load(tensors[0][0])
    assert np.array_equal(gate.decode(), oracle.bin_decode(*refs["gate"], 64, 256))
    up = cat.load(tensors[1][0])
    assert np.array_equal(up.decode(), _rice_dense(oracle, refs["up"]))
    down = cat.load(tensors[2][0])
    x = oracle.deterministic_input(256)
    L, R = refs["down"]
    assert oracle.relative_l2(down.matvec(x), oracle.hgravs01_matvec(L, R, 96, 32, 256, x, 3, 64)) < TOL
    lm = cat.load(tensors[3][0])
    assert np.array_equal(lm.decode(), oracle.uniform_decode(*refs["lm"], 40, 128, 8, 64))


def test_catalog_rejects_corruption(ctx, oracle, tmp_path):
    from hawking_amd._lib import HawkingError
    from hawking_amd.containers import MixedCatalog
    INV, GEO, _, _ = _codes()
    tensors, _ = _catalog_tensors(oracle)
    mpath = W.write_catalog(tmp_path, tensors)
    cat = MixedCatalog(ctx, str(mpath))
    with pytest.raises(HawkingError) as e:
        cat.record("model.layers.9.nope")
    assert e.value.code == INV
    # one flipped payload byte: caught by the SHA-256 check, not without it
    name = tensors[0][0]
    rec = cat.record(name)
    seg = tmp_path / "segments" / f"segment_{rec['segment_id']:03d}.bin"
    cat.close()
    raw = bytearray(seg.read_bytes())
    raw[rec["offset"] + rec["nbytes"] - 1] ^= 0x01   # the last sign byte
    seg.write_bytes(bytes(raw))
    cat = MixedCatalog(ctx, str(mpath))
    say("catalog sha mismatch")
    with pytest.raises(HawkingError) as e:
        cat.load(name)
    assert e.value.code == GEO
    cat.load(name, verify=False)
    cat.close()
    # a catalog that does not match the manifest's digest
    cpath = tmp_path / "catalog.hq80m15"
    craw = bytearray(cpath.read_bytes())
    craw[-1] ^= 0x20
    cpath.write_bytes(bytes(craw))
    with pytest.raises(HawkingError) as e:
        MixedCatalog(ctx, str(mpath))
    assert e.value.code == INV
    # a duplicate tensor name, with the manifest digest updated
    dup = tmp_path / "dup"
    dup.mkdir()
    t = tensors[3]
    mdup = W.write_catalog(dup, [t, (t[0], t[1], t[2], t[3], t[4])])
    with pytest.raises(HawkingError) as e:
        MixedCatalog(ctx, str(mdup))
    assert e.value.code == GEO
    # wrong manifest schema
    m = json.loads(mpath.read_text())
    m["schema"] = "something.else"
    (tmp_path / "bad.json").write_text(json.dumps(m))
    with pytest.raises(HawkingError) as e:
        MixedCatalog(ctx, str(tmp_path / "bad.json"))
    assert e.value.code == INV
