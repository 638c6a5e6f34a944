"""GPU parity of HGRAVR02 organs (binary base + Rice-coded 1-bit residual)
against the CPU oracle, through the C ABI.

Bars: the device packer, the bind-time expand (via the decode probe) and the
residual apply given the same base are bit-exact; the full matvec is within
2e-5 relative L2 of the oracle's serial f32 binary_rice_q1_matvec_f32 and of
the FP64 authority.
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


def _organ(ctx, p):
    from hawking_amd.organs import RiceQ1Packed
    return RiceQ1Packed(ctx, p.rows, p.cols, p.bin_scales, p.bin_signs, p.first, p.rice_k, p.rice, p.count,
                        p.res_scale, p.res_signs)


def _dense(oracle, p):
    d = oracle.bin_decode(p.bin_scales, p.bin_signs, p.rows, p.cols).reshape(-1).copy()
    s = oracle.f16_to_f32(p.res_scale)
    bits = np.unpackbits(p.res_signs, bitorder="little")[:p.count]
    np.add.at(d, p.indices.astype(np.int64), np.where(bits == 1, s, -s).astype(np.float32))
    return d.reshape(p.rows, p.cols)


def _weights(oracle, rows, cols, tag):
    if tag == "det":
        return oracle.deterministic_matrix(rows, cols, 11)
    return oracle.normal(oracle.stream_key(U.SEED, 0xA2 + rows * 7 + cols), rows * cols, 0.02).reshape(rows, cols)


@pytest.mark.parametrize("rows,cols,tag", [(8, 128, "det"), (512, 2048, "n"), (2048, 512, "n"), (37, 384, "n")])
def test_rice_organ_matvec_and_decode(ctx, oracle, rows, cols, tag):
    w = _weights(oracle, rows, cols, tag)
    x = oracle.deterministic_input(cols) if tag == "det" else \
        oracle.normal(oracle.stream_key(U.SEED, 0xA3 + rows), cols, 1.0)
    p = oracle.rice_q1_pack(w, rows, cols, 0.02)
    say("rice organ", rows, cols, tag, "outliers", p.count)
    o = _organ(ctx, p)
    assert np.array_equal(o.decode(), _dense(oracle, p))
    y = o.matvec(x)
    assert oracle.relative_l2(y, oracle.rice_q1_matvec(p, x)) < TOL
    assert oracle.relative_l2(y, oracle.rice_q1_matvec_f64(p, x)) < TOL
    n = rows * cols
    assert o.packed_bytes == n // 8 + n // 64 + 4 + p.rice.size + 2 + (p.count + 7) // 8


@pytest.mark.parametrize("rows,cols", [(8, 128), (512, 2048), (300, 1024)])
def test_rice_residual_apply_is_bit_exact(ctx, oracle, rows, cols):
    """Given the oracle's serial binary result, y += residual x equals the
    reference's serial correction bit for bit (index order per row)."""
    w = _weights(oracle, rows, cols, "n")
    x = oracle.normal(oracle.stream_key(U.SEED, 0xA4 + rows), cols, 1.0)
    p = oracle.rice_q1_pack(w, rows, cols, 0.05)
    say("rice apply", rows, cols, "outliers", p.count)
    o = _organ(ctx, p)
    y0 = oracle.bin_matvec(p.bin_scales, p.bin_signs, rows, cols, x)
    yd = ctx.to_device(y0)
    o.apply_residual_device(ctx.to_device(x), yd)
    assert np.array_equal(yd.download(), oracle.rice_q1_apply(p, x, y0))
    assert np.array_equal(oracle.rice_q1_apply(p, x, y0), oracle.rice_q1_matvec(p, x))


def _tie_weights(rows, cols, seed):
    rng = np.random.default_rng(seed)
    return (rng.integers(-8, 9, (rows, cols)) / 8.0).astype(np.float32)


@pytest.mark.parametrize("case", ["kat", "det", "normal", "ties", "ratio_small", "ratio_max"])
def test_device_rice_packer_bit_exact(ctx, oracle, case):
    from hawking_amd import organs
    ratio = 0.02
    if case == "kat":
        rows, cols = 1, 128
        w = np.ones((1, 128), np.float32)
        w[0, 5], w[0, 9], w[0, 77] = 3.0, -2.0, 3.0
    elif case == "det":
        rows, cols = 8, 128
        w = oracle.deterministic_matrix(rows, cols, 11)
    elif case == "ties":
        rows, cols = 64, 1024
        w = _tie_weights(rows, cols, 5)
    else:
        rows, cols = 512, 2048
        w = _weights(oracle, rows, cols, "n")
        ratio = {"normal": 0.02, "ratio_small": 0.0004, "ratio_max": 0.1}[case]
    say("rice pack", case, rows, cols, ratio)
    src, bufs = organs.pack_binary_rice_device(ctx, ctx.to_device(w), rows, cols, ratio)
    p = oracle.rice_q1_pack(w, rows, cols, ratio)
    assert (src.outlier_count, src.first_index, src.rice_k, src.residual_scale_f16) == \
        (p.count, p.first, p.rice_k, p.res_scale)
    assert src.rice_bytes == p.rice.size
    assert np.array_equal(bufs[0].download(), p.bin_scales)
    assert np.array_equal(bufs[1].download(), p.bin_signs)
    assert np.array_equal(bufs[2].download(), p.res_signs)
    assert np.array_equal(bufs[3].download()[:p.rice.size], p.rice)
    # the device body binds to an organ equal to the oracle-packed one
    o = organs.RiceQ1Packed.from_device(ctx, src)
    assert np.array_equal(o.decode(), _dense(oracle, p))


def test_synthetic_rice_organ_matches_oracle(ctx, oracle):
    from hawking_amd._lib import HK_BIN_RICE
    from hawking_amd.organs import SyntheticOrgan
    rows, cols = 96, 512
    key = oracle.stream_key(U.SEED, 0xA5)
    say("synthetic rice", rows, cols)
    o = SyntheticOrgan(ctx, HK_BIN_RICE, rows, cols, key, 0, group=128, sigma=0.02)
    p = oracle.rice_q1_pack(oracle.normal(key, rows * cols, 0.02), rows, cols, 0.02)
    assert np.array_equal(o.decode(), _dense(oracle, p))


def test_rice_organ_set_matches_single(ctx, oracle):
    from hawking_amd.organs import OrganSet
    rows, cols, n = 256, 1024, 5
    ps, xs = [], []
    for i in range(n):
        w = oracle.normal(oracle.stream_key(U.SEED, 0xA6 + i), rows * cols, 0.02).reshape(rows, cols)
        ps.append(oracle.rice_q1_pack(w, rows, cols, 0.02))
        xs.append(oracle.normal(oracle.stream_key(U.SEED, 0xA7 + i), cols, 1.0))
    say("rice set", n, rows, cols)
    orgs = [_organ(ctx, p) for p in ps]
    s = OrganSet(ctx, orgs)
    x = ctx.to_device(np.stack(xs))
    y = ctx.empty((n, rows))
    s.gemv(x, cols, y, rows)
    yy = y.download()
    for i in range(n):
        assert np.array_equal(yy[i], orgs[i].matvec(xs[i]))
        assert oracle.relative_l2(yy[i], oracle.rice_q1_matvec(ps[i], xs[i])) < TOL


@pytest.mark.parametrize("n", [521, 3100])
def test_rice_organ_set_large_matches_single(ctx, oracle, n):
    # large HGRAVR02 sets (the streamed launch shapes): the same bits as one organ at a time
    from hawking_amd._lib import HK_BIN_RICE
    from hawking_amd.organs import OrganSet, SyntheticOrgan
    rows, cols = 32, 256
    say("rice set large", n, rows, cols)
    orgs = [SyntheticOrgan(ctx, HK_BIN_RICE, rows, cols, oracle.stream_key(U.SEED, (0xA8 << 20) + i), 0, group=128,
                           sigma=0.02) for i in range(n)]
    s = OrganSet(ctx, orgs)
    xs = np.stack([oracle.normal(oracle.stream_key(U.SEED, (0xA9 << 20) + i), cols, 1.0) for i in range(n)])
    x = ctx.to_device(xs)
    y = ctx.empty((n, rows))
    s.gemv(x, cols, y, rows)
    y1 = y.download()
    s.gemv(x, cols, y, rows)  # a second call gives the same bits
    assert np.array_equal(y.download(), y1)
    for i in sorted({0, 1, n // 3, n // 2, n // 2 + 1, n - 2, n - 1}):
        assert np.array_equal(y1[i], orgs[i].matvec(xs[i])), i


@pytest.mark.parametrize("rows,cols,n", [(512, 2048, 520), (2048, 512, 130)])
def test_rice_organ_set_fused_matches_single(ctx, oracle, rows, cols, n):
    # sets of >= 16,384 row tiles take the GEMV with the residual in its
    # epilogue (256 rows a workgroup for 2048 columns, 512 for 512): the same
    # bits as the GEMV followed by the apply, one organ at a time
    from hawking_amd._lib import HK_BIN_RICE
    from hawking_amd.organs import OrganSet, SyntheticOrgan
    say("rice set fused", n, rows, cols)
    orgs = [SyntheticOrgan(ctx, HK_BIN_RICE, rows, cols, oracle.stream_key(U.SEED, (0xAA << 20) + i), 0, group=128,
                           sigma=0.02) for i in range(n)]
    s = OrganSet(ctx, orgs)
    xs = np.stack([oracle.normal(oracle.stream_key(U.SEED, (0xAB << 20) + i), cols, 1.0) for i in range(n)])
    x = ctx.to_device(xs)
    y = ctx.empty((n, rows))
    s.gemv(x, cols, y, rows)
    y1 = y.download()
    s.gemv(x, cols, y, rows)
    assert np.array_equal(y.download(), y1)
    for i in range(n):
        assert np.array_equal(y1[i], orgs[i].matvec(xs[i])), i


def test_rice_fused_byte_steps_edge_rows(ctx, oracle):
    """The fused GEMV's byte-step records (one byte per step through the
    three-entry product table) at their edges: a row's first outlier at
    column 0, gaps of 85, 86 and 2,047 columns (zero, one and 24 steps through
    -0 entries), adjacent columns, a row ending at the last column (padding
    steps past it), and rows without outliers.  512 organs of 512 x 2048 reach
    the fused launch (16,384 row tiles); its sums must be the GEMV-then-apply
    sums of each organ, bit for bit."""
    rows, cols, n = 512, 2048, 512
    pattern = [[0, 2047], [], [1, 86, 172, 173, 2046], list(range(100, 140))]
    planted = []
    for r in range(rows):
        planted += [r * cols + c for c in pattern[r % 4]]
    rng = np.random.default_rng(7)
    w = (rng.standard_normal(rows * cols) * 1e-3).astype(np.float32)
    w[planted] = np.where(rng.random(len(planted)) < 0.5, -1.0, 1.0).astype(np.float32)
    ratio = len(planted) / (rows * cols)  # a power-of-two denominator: the count is exact
    p = oracle.rice_q1_pack(w.reshape(rows, cols), rows, cols, ratio)
    say("rice byte steps", rows, cols, n, "outliers", p.count)
    assert p.count == len(planted) and set(p.indices.tolist()) == set(planted)
    from hawking_amd.organs import OrganSet
    orgs = [_organ(ctx, p) for _ in range(n)]
    s = OrganSet(ctx, orgs)
    xs = np.stack([oracle.normal(oracle.stream_key(U.SEED, (0xAC << 20) + i), cols, 1.0) for i in range(n)])
    y = ctx.empty((n, rows))
    s.gemv(ctx.to_device(xs), cols, y, rows)
    yy = y.download()
    for i in (0, 1, n // 2, n - 1):
        assert np.array_equal(yy[i], orgs[i].matvec(xs[i])), i
        assert oracle.relative_l2(yy[i], oracle.rice_q1_matvec(p, xs[i])) < TOL


def test_rice_upload_rejects_bad_streams(ctx, oracle):
    from hawking_amd._lib import HK_E_GEOMETRY, HK_E_NONFINITE, HawkingError
    from hawking_amd.organs import RiceQ1Packed
    rows, cols = 16, 256
    p = oracle.rice_q1_pack(_weights(oracle, rows, cols, "n"), rows, cols, 0.05)
    base = dict(rows=rows, cols=cols, bin_scales=p.bin_scales, bin_signs=p.bin_signs, first_index=p.first,
                rice_k=p.rice_k, rice=p.rice, outlier_count=p.count, residual_scale_f16=p.res_scale,
                residual_signs=p.res_signs)
    cases = [(dict(rice=p.rice[:p.rice.size // 2]), HK_E_GEOMETRY),          # overrun
             (dict(first_index=rows * cols), HK_E_GEOMETRY),                # first index past the organ
             (dict(outlier_count=0), HK_E_GEOMETRY),
             (dict(residual_scale_f16=0x7C00), HK_E_NONFINITE),
             (dict(cols=200), HK_E_GEOMETRY)]
    bad_scales = p.bin_scales.copy()
    bad_scales[3] = 0x7E00
    cases.append((dict(bin_scales=bad_scales), HK_E_NONFINITE))
    for change, code in cases:
        say("rice reject", sorted(change))
        with pytest.raises(HawkingError) as e:
            RiceQ1Packed(ctx, **{**base, **change})
        assert e.value.code == code, change
