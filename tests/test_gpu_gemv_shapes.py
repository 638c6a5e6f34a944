"""GEMV over organ sets in every launch shape the dispatcher picks, and x
images of several quantization rounds, against the oracle (through the C ABI).

The dispatcher sizes the launch by the set's total row tiles: >= 16384 tiles
(the streamed shapes of the benchmark, as tiles per wave group / steps in
flight / tiles per workgroup: binary 4 / 3 / 16 with >= 4 steps, else
2 / 3 / 32; Q4 2 / 3 / 16; mixed 1 / 3 / 16), >= 4096 (2 / 2 / 8) and below
(1 / 2 / 4 or 1).  The x image is built 2048 columns per
round; organs wider than 2048 columns take several rounds, and beyond 8192
columns the later rounds re-read x.  Organs are generated on the device; the
oracle regenerates the ones it checks (first, middle, last) bit-identically.
Bar: 2e-5 relative L2 against the oracle's serial f32 matvec.
"""
import sys

import numpy as np
import pytest

from tests import hk_testutil as U

pytestmark = pytest.mark.gpu
TOL = 2e-5
HK_Q4, HK_BIN, HK_MIXED, HK_Q8, HK_U3, HK_BIN_RICE = U.HK_Q4, U.HK_BIN, U.HK_MIXED, 4, 5, 6


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    from hawking_amd.runtime import Context
    return Context(0)


def _keys(oracle, tag, i):
    sid = (0x5E7 << 40) | (tag << 24) | i
    return oracle.stream_key(U.SEED, sid), oracle.stream_key(U.SEED, sid ^ (1 << 39))


def _oracle_matvec(oracle, kind, group, rows, cols, key, coin_key, x):
    w = oracle.normal(key, rows * cols, U.SIGMA_W).reshape(rows, cols)
    if kind == HK_BIN:
        s, g = oracle.bin_pack(w)
        return oracle.bin_matvec(s, g, rows, cols, x)
    if kind == HK_Q4:
        s, c = oracle.q4_pack(w, group)
        return oracle.q4_matvec(s, c, rows, cols, group, x)
    if kind == HK_Q8:
        s, c = oracle.uniform_pack(w, rows, cols, 8, 64)
        return oracle.uniform_matvec(s, c, rows, cols, x, 8, 64)
    m = oracle.mixed_pack(w, oracle.mixed_coins(coin_key, rows * cols // 128))
    return oracle.mixed_matvec(m, x)


CASES = [
    # label, kind, group, rows, cols, n organs
    ("bin streamed 16/wg", HK_BIN, 128, 512, 2048, 512),
    ("bin streamed 32/wg", HK_BIN, 128, 2048, 512, 128),
    ("q4 streamed", HK_Q4, 32, 512, 2048, 512),
    ("mixed streamed", HK_MIXED, 128, 512, 2048, 512),
    ("bin streamed 2-tile", HK_BIN, 128, 1024, 1536, 256),
    ("bin mid", HK_BIN, 128, 512, 2048, 128),
    ("mixed mid ragged", HK_MIXED, 128, 500, 1024, 140),
    ("q4 small", HK_Q4, 64, 96, 1024, 5),
    ("bin 3 rounds", HK_BIN, 128, 48, 6144, 3),
    ("bin 5 rounds (re-read)", HK_BIN, 128, 40, 10240, 2),
    ("mixed 4 rounds", HK_MIXED, 128, 33, 7168, 2),
    ("q4 5 rounds (re-read)", HK_Q4, 128, 24, 9216, 2),
    ("q8 streamed", HK_Q8, 64, 512, 2048, 512),
    ("q8 mid ragged", HK_Q8, 64, 300, 1024, 240),
    ("q8 small", HK_Q8, 64, 40, 704, 3),
    ("q8 5 rounds (re-read)", HK_Q8, 64, 24, 9216, 2),
]


@pytest.mark.parametrize("label,kind,group,rows,cols,n", CASES, ids=[c[0] for c in CASES])
def test_organ_set_launch_shapes(ctx, oracle, label, kind, group, rows, cols, n):
    from hawking_amd import organs
    say(label, kind, group, rows, cols, n)
    tag = CASES.index((label, kind, group, rows, cols, n))
    keys = [_keys(oracle, tag, i) for i in range(n)]
    orgs = [organs.SyntheticOrgan(ctx, kind, rows, cols, k, ck, group=group) for k, ck in keys]
    oset = organs.OrganSet(ctx, orgs)
    rng = np.random.default_rng(1000 + tag)
    xs = rng.standard_normal((n, cols)).astype(np.float32)
    ys = (rows + 3) // 4 * 4                       # y rows 16-byte aligned
    y = ctx.empty((n, ys))
    oset.gemv(ctx.to_device(xs), cols, y, ys)
    yg = y.download()[:, :rows]
    for i in sorted({0, n // 2, n - 1}):
        k, ck = keys[i]
        ref = _oracle_matvec(oracle, kind, group, rows, cols, k, ck, xs[i])
        err = oracle.relative_l2(yg[i], ref)
        assert err < TOL, (label, i, err)


def test_organ_wider_than_lds_image_is_rejected(ctx):
    from hawking_amd import organs
    from hawking_amd._lib import HK_E_GEOMETRY, HawkingError
    with pytest.raises(HawkingError) as e:
        organs.SyntheticOrgan(ctx, HK_BIN, 16, 16384, 1, 2)
    assert e.value.code == HK_E_GEOMETRY


def _oracle_decode(oracle, kind, group, rows, cols, key, coin_key):
    """The oracle's pack of the same draws, decoded, and its canonical byte count."""
    w = oracle.normal(key, rows * cols, U.SIGMA_W).reshape(rows, cols)
    if kind == HK_BIN:
        s, g = oracle.bin_pack(w)
        return oracle.bin_decode(s, g, rows, cols), s.nbytes + g.nbytes
    if kind == HK_Q4:
        s, c = oracle.q4_pack(w, group)
        return oracle.q4_decode(s, c, rows, cols, group), s.nbytes + c.nbytes
    if kind == HK_Q8:
        s, c = oracle.uniform_pack(w, rows, cols, 8, 64)
        return oracle.uniform_decode(s, c, rows, cols, 8, 64), s.nbytes + c.nbytes
    if kind == HK_U3:
        s, c = oracle.uniform_pack(w, rows, cols, 3, 64)
        return oracle.uniform_decode(s, c, rows, cols, 3, 64), s.nbytes + c.nbytes
    if kind == HK_BIN_RICE:
        # base + (+-scale) at each outlier, in f32 (hk_decode_rows of an HGRAVR02 organ)
        p = oracle.rice_q1_pack(w, rows, cols, 0.02)
        d = oracle.bin_decode(p.bin_scales, p.bin_signs, rows, cols).reshape(-1).copy()
        sc = oracle.f16_to_f32(p.res_scale)
        bits = np.unpackbits(p.res_signs, bitorder="little")[:p.count]
        np.add.at(d, p.indices.astype(np.int64), np.where(bits == 1, sc, -sc).astype(np.float32))
        # canonical HGRAVR02 body: base, first_index (u32), Rice stream, f16 scale, sign bits
        nbytes = p.bin_scales.nbytes + p.bin_signs.nbytes + 4 + p.rice.nbytes + 2 + p.res_signs.nbytes
        return d, nbytes
    m = oracle.mixed_pack(w, oracle.mixed_coins(coin_key, rows * cols // 128))
    return oracle.mixed_decode(m), m.nbytes()


SYNTH = [
    ("q4 g32", HK_Q4, 32, 512, 2048),
    ("q4 g64", HK_Q4, 64, 48, 1024),
    ("q4 g128", HK_Q4, 128, 40, 640),
    ("bin 512x2048", HK_BIN, 128, 512, 2048),
    ("bin 2048x512", HK_BIN, 128, 2048, 512),
    ("mixed 512x2048", HK_MIXED, 128, 512, 2048),
    ("mixed 2048x512", HK_MIXED, 128, 2048, 512),
    ("mixed ragged", HK_MIXED, 128, 33, 1152),
    ("q8 512x2048", HK_Q8, 64, 512, 2048),
    # the mixed-1p5 model's HGRAVR02 up and HGRAVS01 factors (2 % outliers; flat 3-bit groups)
    ("rice 512x2048", HK_BIN_RICE, 128, 512, 2048),
    ("u3 2048x160", HK_U3, 64, 2048, 160),
    ("u3 160x512", HK_U3, 64, 160, 512),
]


@pytest.mark.parametrize("label,kind,group,rows,cols", SYNTH, ids=[c[0] for c in SYNTH])
def test_synthetic_organ_decodes_bit_exact(ctx, oracle, label, kind, group, rows, cols):
    """hk_organ_synthetic (device draws, device packer, load-time repack: the
    path that builds the benchmark's organs and the config-4 model) decodes
    bit for bit to the oracle's pack of the same draws (hk_decode_rows), and
    reports the oracle's canonical byte count."""
    from hawking_amd import organs
    say("synthetic decode", label)
    tag = 0x400 + SYNTH.index((label, kind, group, rows, cols))
    k, ck = _keys(oracle, tag, 0)
    o = organs.SyntheticOrgan(ctx, kind, rows, cols, k, ck, group=group)
    want, nbytes = _oracle_decode(oracle, kind, group, rows, cols, k, ck)
    got = o.decode()
    assert np.array_equal(got.view(np.uint32), np.asarray(want, np.float32).reshape(rows, cols).view(np.uint32))
    assert o.packed_bytes == nbytes
