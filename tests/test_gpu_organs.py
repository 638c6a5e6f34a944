"""GPU parity of the packed organs against the CPU oracle (through the C ABI).

Bars: the generator, the device packers and the decode probe are bit-exact;
matvec outputs are within 2e-5 relative L2 of the oracle's serial f32 path
and of the FP64 authority.
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


# ------------------------------------------------------------------ generator / packers

def test_generator_is_bit_identical_to_oracle(ctx, oracle):
    from hawking_amd import organs
    for sid, n, sigma in [(1, 100003, 0.02), (U.stream_id(3, 7, 1), 4096, 1.0)]:
        say("synth_normal", sid, n, sigma)
        key = oracle.stream_key(U.SEED, sid)
        assert organs.stream_key(U.SEED, sid) == key
        got = organs.synth_normal(ctx, key, n, sigma).download()
        assert np.array_equal(got.view(np.uint32), oracle.normal(key, n, sigma).view(np.uint32))


def _edge_weights(rng, rows, cols):
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[0, :] = 0.0                                  # all-zero groups
    w[1, :32] = np.arange(32, dtype=np.float32) - 16  # exact ties at x.5 after scaling
    w[1, 32:64] = 1e-7                             # f16-subnormal scales
    w[2, ::3] = -0.0
    return w


@pytest.mark.parametrize("group", [32, 64, 128])
def test_device_q4_packer_bit_exact(ctx, oracle, group):
    from hawking_amd import organs
    rng = np.random.default_rng(group)
    w = _edge_weights(rng, 64, 512)
    say("pack_q4", w.shape, group)
    s, c = organs.pack_q4_device(ctx, ctx.to_device(w), 64, 512, group)
    rs, rc = oracle.q4_pack(w, group)
    assert np.array_equal(s.download(), rs) and np.array_equal(c.download(), rc)


def test_device_binary_packer_bit_exact(ctx, oracle):
    from hawking_amd import organs
    rng = np.random.default_rng(7)
    w = _edge_weights(rng, 32, 1024)
    v0 = np.float32(2.0**-14 * (1 + 2.0**-11))   # double-rounding case
    w[3, :128] = v0
    w[3, 0] = np.nextafter(v0, np.float32(1))
    say("pack_bin", w.shape)
    s, g = organs.pack_binary_group_device(ctx, ctx.to_device(w), 32, 1024)
    rs, rg = oracle.bin_pack(w)
    assert np.array_equal(s.download(), rs) and np.array_equal(g.download(), rg)


def test_device_q2_packer_bit_exact(ctx, oracle):
    from hawking_amd import organs
    rng = np.random.default_rng(8)
    w = _edge_weights(rng, 16, 512).reshape(-1)
    w[4096:4160] = np.linspace(-1.5, 1.5, 64, dtype=np.float32)
    say("pack_q2", w.size)
    s, c = organs.pack_q2_device(ctx, ctx.to_device(w), w.size)
    rs, rc = oracle.q2_pack(w)
    assert np.array_equal(s.download(), rs) and np.array_equal(c.download(), rc)


def test_device_q8_packer_bit_exact(ctx, oracle):
    from hawking_amd import organs
    rng = np.random.default_rng(8)
    w = _edge_weights(rng, 64, 512)
    d = 1.0 + 2.0 ** -11
    w[3, :4] = [127 * d, 62.5 * d, 62.5, -62.5 * d]     # half-away rounding, f32 divisor
    w[3, 4:64] = 0.0
    say("pack_q8", w.shape)
    s, c = organs.pack_q8_device(ctx, ctx.to_device(w), 64, 512)
    rs, rc = oracle.uniform_pack(w, 64, 512, 8, 64)
    assert np.array_equal(s.download(), rs) and np.array_equal(c.download(), rc)


def test_device_packer_rejects_nonfinite(ctx):
    from hawking_amd import organs
    from hawking_amd._lib import HK_E_NONFINITE, HawkingError
    w = np.zeros((4, 128), np.float32)
    w[2, 5] = np.nan
    with pytest.raises(HawkingError) as e:
        organs.pack_q4_device(ctx, ctx.to_device(w), 4, 128, 32)
    assert e.value.code == HK_E_NONFINITE


# ------------------------------------------------------------------ organs

def _q4(ctx, oracle, w, group):
    from hawking_amd.organs import Qwen80Q4PackedTensor
    s, c = oracle.q4_pack(w, group)
    return Qwen80Q4PackedTensor(ctx, s, c, w.shape[0], w.shape[1], group), (s, c)


def _bin(ctx, oracle, w):
    from hawking_amd.organs import BinaryGroupPacked
    s, g = oracle.bin_pack(w)
    return BinaryGroupPacked(ctx, s, g, w.shape[0], w.shape[1]), (s, g)


def _mixed(ctx, oracle, w, sel):
    from hawking_amd.organs import MixedPackedTensor
    m = oracle.mixed_pack(w, sel)
    return MixedPackedTensor(ctx, w.shape[0], w.shape[1], m.tags, m.bin_scales, m.bin_signs, m.q2_scales,
                             m.q2_codes), m


def test_config1_q4_512x2048_g32(ctx, oracle):
    key = oracle.stream_key(U.SEED, 0xC1)
    w = oracle.normal(key, 512 * 2048, 0.02).reshape(512, 2048)
    x = oracle.normal(oracle.stream_key(U.SEED, 0xC1 + 1), 2048, 1.0)
    say("config1 q4 512x2048 g32")
    organ, (s, c) = _q4(ctx, oracle, w, 32)
    assert organ.packed_bytes == 589_824
    assert np.array_equal(organ.decode(), oracle.q4_decode(s, c, 512, 2048, 32))
    y = organ.matvec(x)
    yo = oracle.q4_matvec(s, c, 512, 2048, 32, x)
    y64 = oracle.q4_matvec_f64(s, c, 512, 2048, 32, x)
    assert oracle.relative_l2(y, yo) < TOL
    assert oracle.relative_l2(y, y64) < TOL


@pytest.mark.parametrize("shape", [(512, 2048), (2048, 512)])
def test_config2_binary(ctx, oracle, shape):
    rows, cols = shape
    w = oracle.normal(oracle.stream_key(U.SEED, 0xC2 + rows), rows * cols, 0.02).reshape(rows, cols)
    x = oracle.normal(oracle.stream_key(U.SEED, 0xC2 + rows + 1), cols, 1.0)
    say("config2 binary", shape)
    organ, (s, g) = _bin(ctx, oracle, w)
    assert organ.packed_bytes == 147_456
    assert np.array_equal(organ.decode(), oracle.bin_decode(s, g, rows, cols))
    y = organ.matvec(x)
    assert oracle.relative_l2(y, oracle.bin_matvec(s, g, rows, cols, x)) < TOL
    assert oracle.relative_l2(y, oracle.bin_matvec_f64(s, g, rows, cols, x)) < TOL


@pytest.mark.parametrize("shape", [(512, 2048), (2048, 512), (13, 384)])
def test_mixed_organ(ctx, oracle, shape):
    rows, cols = shape
    w = oracle.normal(oracle.stream_key(U.SEED, 0xC4 + rows), rows * cols, 0.02).reshape(rows, cols)
    sel = oracle.mixed_coins(oracle.stream_key(U.SEED, 0xC4 + rows + 7), rows * cols // 128)
    x = oracle.normal(oracle.stream_key(U.SEED, 0xC4 + rows + 1), cols, 1.0)
    say("mixed organ", shape)
    organ, m = _mixed(ctx, oracle, w, sel)
    assert np.array_equal(organ.decode(), oracle.mixed_decode(m))
    y = organ.matvec(x)
    assert oracle.relative_l2(y, oracle.mixed_matvec(m, x)) < TOL
    assert oracle.relative_l2(y, oracle.mixed_matvec_f64(m, x)) < TOL


@pytest.mark.parametrize("kinds", ["q2", "binary", "coin"])
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_mixed_organ_extreme_x(ctx, oracle, kinds, sign):
    # every |x| near max|x| (fixed-point X within 0.1 % of 2^23), the Q2 top
    # field's columns (6, 7 of every 8) of the opposite sign: the largest
    # magnitudes the engine's exact int32 corrections 3 sum X - 4 sum_top X reach
    rows, cols = 96, 1024
    w = oracle.normal(oracle.stream_key(U.SEED, 0xC4E0), rows * cols, 0.02).reshape(rows, cols)
    groups = rows * cols // 128
    sel = {"q2": np.zeros(groups, np.uint8), "binary": np.ones(groups, np.uint8),
           "coin": oracle.mixed_coins(oracle.stream_key(U.SEED, 0xC4E1), groups)}[kinds]
    c = np.arange(cols)
    x = (sign * np.where(c % 8 < 6, 0.999, -0.999) * (1.0 - 1e-4 * (c % 5))).astype(np.float32)
    say("mixed organ extreme x", kinds, sign)
    organ, m = _mixed(ctx, oracle, w, sel)
    y = organ.matvec(x)
    assert oracle.relative_l2(y, oracle.mixed_matvec(m, x)) < TOL
    assert oracle.relative_l2(y, oracle.mixed_matvec_f64(m, x)) < TOL


def _q8(ctx, oracle, w):
    from hawking_amd.organs import UniformFactorPacked
    s, c = oracle.uniform_pack(w, w.shape[0], w.shape[1], 8, 64)
    return UniformFactorPacked(ctx, s, c, w.shape[0], w.shape[1]), (s, c)


@pytest.mark.parametrize("shape", [(512, 2048), (2048, 512), (13, 384), (1, 7168)])
def test_uniform_q8_organ(ctx, oracle, shape):
    """HGRAVU01 (q8, group 64): decode bit-exact, matvec vs the serial f32
    oracle and the FP64 authority."""
    rows, cols = shape
    w = oracle.normal(oracle.stream_key(U.SEED, 0xC8 + rows), rows * cols, 0.02).reshape(rows, cols)
    x = oracle.normal(oracle.stream_key(U.SEED, 0xC8 + rows + 1), cols, 1.0)
    say("uniform q8 organ", shape)
    organ, (s, c) = _q8(ctx, oracle, w)
    assert organ.packed_bytes == rows * cols + rows * cols // 64 * 2
    assert np.array_equal(organ.decode(), oracle.uniform_decode(s, c, rows, cols, 8, 64))
    y = organ.matvec(x)
    assert oracle.relative_l2(y, oracle.uniform_matvec(s, c, rows, cols, x, 8, 64)) < TOL
    assert oracle.relative_l2(y, oracle.uniform_matvec_f64(s, c, rows, cols, x, 8, 64)) < TOL


def test_uniform_q8_rejects_bad_geometry(ctx, oracle):
    from hawking_amd._lib import HK_E_GEOMETRY, HawkingError
    from hawking_amd.organs import UniformFactorPacked
    s, c = oracle.uniform_pack(np.ones((2, 96), np.float32), 2, 96, 8, 64)
    with pytest.raises(HawkingError) as e:
        UniformFactorPacked(ctx, s, c[:192], 2, 96)
    assert e.value.code == HK_E_GEOMETRY


def _u3(ctx, oracle, w):
    from hawking_amd.organs import UniformFactor3
    s, c = oracle.uniform_pack(w, w.shape[0], w.shape[1], 3, 64)
    return UniformFactor3(ctx, s, c, w.shape[0], w.shape[1]), (s, c)


@pytest.mark.parametrize("count", [64 * 37, 1000])
def test_device_u3_packer_bit_exact(ctx, oracle, count):
    """3-bit factor packer (HGRAVS01 body): whole groups and a ragged last group."""
    from hawking_amd import organs
    rng = np.random.default_rng(count)
    w = (rng.standard_normal(count) * 0.02).astype(np.float32)
    d = 1.0 + 2.0 ** -11
    w[:5] = [3 * d, 1.5 * d, -1.5 * d, 0.5 * d, 1.5]    # half-away ties under the f32 divisor
    w[64:128] = 0.0                                     # an all-zero group
    say("pack_u3", count)
    s, c = organs.pack_u3_device(ctx, ctx.to_device(w), count)
    rs, rc = oracle.uniform_pack(w, 1, count, 3, 64)
    assert np.array_equal(s.download(), rs) and np.array_equal(c.download(), rc)


@pytest.mark.parametrize("shape", [(2048, 160), (160, 2048), (13, 96), (16, 32), (1, 6144), (40, 224)])
def test_uniform_u3_factor_organ(ctx, oracle, shape):
    """HGRAVS01 factor (3-bit, flat 64-groups that may span rows): decode
    bit-exact, matvec vs the serial f32 oracle and the FP64 authority."""
    rows, cols = shape
    w = oracle.normal(oracle.stream_key(U.SEED, 0xD3 + rows), rows * cols, 0.02).reshape(rows, cols)
    x = oracle.normal(oracle.stream_key(U.SEED, 0xD3 + rows + 1), cols, 1.0)
    say("uniform u3 factor", shape)
    organ, (s, c) = _u3(ctx, oracle, w)
    groups = (rows * cols + 63) // 64
    assert organ.packed_bytes == groups * 26
    assert np.array_equal(organ.decode(), oracle.uniform_decode(s, c, rows, cols, 3, 64))
    y = organ.matvec(x)
    assert oracle.relative_l2(y, oracle.uniform_matvec(s, c, rows, cols, x, 3, 64)) < TOL
    assert oracle.relative_l2(y, oracle.uniform_matvec_f64(s, c, rows, cols, x, 3, 64)) < TOL


@pytest.mark.parametrize("rows,rank,cols,n", [(2048, 160, 768, 6), (512, 96, 2048, 5), (48, 32, 4096, 3)])
def test_hgravs01_set_one_launch_matches_two_launches(ctx, oracle, rows, rank, cols, n):
    """hk_gemv_lowrank_set (one workgroup per pair, mid on chip) gives the
    same bits as the two set launches through a mid buffer, and stays within
    tolerance of the oracle's two-stage matvec and the FP64 product."""
    from hawking_amd.organs import OrganSet, gemv_lowrank_set
    say("hgravs01 set", rows, rank, cols, n)
    lefts, rights, packs, xs = [], [], [], []
    for i in range(n):
        key = lambda k: oracle.stream_key(U.SEED, (0xE5 << 20) + (rank << 8) + 16 * i + k)
        Lw = oracle.normal(key(1), rows * rank, 0.05).reshape(rows, rank)
        Rw = oracle.normal(key(2), rank * cols, 0.02).reshape(rank, cols)
        lo, lp = _u3(ctx, oracle, Lw)
        ro, rp = _u3(ctx, oracle, Rw)
        lefts.append(lo)
        rights.append(ro)
        packs.append((lp, rp))
        xs.append(oracle.normal(key(3), cols, 1.0))
    ls, rs = OrganSet(ctx, lefts), OrganSet(ctx, rights)
    xd = ctx.to_device(np.stack(xs))
    y1, mid, y2 = ctx.empty((n, rows)), ctx.empty((n, rank)), ctx.empty((n, rows))
    gemv_lowrank_set(ctx, ls, rs, xd, cols, y1, rows)
    rs.gemv(xd, cols, mid, rank)
    ls.gemv(mid, rank, y2, rows)
    a, b = y1.download(), y2.download()
    assert np.array_equal(a, b)
    y3, mid3 = ctx.empty((n, rows)), ctx.empty((n, rank))
    gemv_lowrank_set(ctx, ls, rs, xd, cols, y3, rows, mid=mid3, mid_stride=rank)
    assert np.array_equal(y3.download(), a) and np.array_equal(mid3.download(), mid.download())
    for i in range(n):
        (ls_, lc), (rs_, rc) = packs[i]
        ref = oracle.hgravs01_matvec((ls_, lc), (rs_, rc), rows, rank, cols, xs[i], 3, 64)
        Ld = oracle.uniform_decode(ls_, lc, rows, rank, 3, 64).astype(np.float64)
        Rd = oracle.uniform_decode(rs_, rc, rank, cols, 3, 64).astype(np.float64)
        assert oracle.relative_l2(a[i], ref) < TOL
        assert oracle.relative_l2(a[i], Ld.reshape(rows, rank) @ (Rd.reshape(rank, cols) @ xs[i].astype(np.float64))) < TOL


def test_hgravs01_set_two_launch_shape_uses_caller_mid(ctx, oracle):
    """A rank above 2048 runs as two set launches through the caller's mid
    workspace (no library scratch); without one the call is refused."""
    from hawking_amd._lib import HK_E_INVALID_ARG, HawkingError
    from hawking_amd.organs import OrganSet, gemv_lowrank_set
    rows, rank, cols, n = 64, 2080, 256, 2
    say("hgravs01 set, two-launch shape", rows, rank, cols)
    lefts, rights, packs, xs = [], [], [], []
    for i in range(n):
        key = lambda k: oracle.stream_key(U.SEED, (0xE6 << 20) + 16 * i + k)
        lo, lp = _u3(ctx, oracle, oracle.normal(key(1), rows * rank, 0.05).reshape(rows, rank))
        ro, rp = _u3(ctx, oracle, oracle.normal(key(2), rank * cols, 0.02).reshape(rank, cols))
        lefts.append(lo)
        rights.append(ro)
        packs.append((lp, rp))
        xs.append(oracle.normal(key(3), cols, 1.0))
    ls, rs = OrganSet(ctx, lefts), OrganSet(ctx, rights)
    xd = ctx.to_device(np.stack(xs))
    y = ctx.empty((n, rows))
    with pytest.raises(HawkingError) as e:
        gemv_lowrank_set(ctx, ls, rs, xd, cols, y, rows)
    assert e.value.code == HK_E_INVALID_ARG
    mid = ctx.empty((n, rank))
    gemv_lowrank_set(ctx, ls, rs, xd, cols, y, rows, mid=mid, mid_stride=rank)
    a = y.download()
    for i in range(n):
        (ls_, lc), (rs_, rc) = packs[i]
        ref = oracle.hgravs01_matvec((ls_, lc), (rs_, rc), rows, rank, cols, xs[i], 3, 64)
        assert oracle.relative_l2(a[i], ref) < TOL


@pytest.mark.parametrize("rows,rank,cols", [(2048, 160, 768), (768, 192, 2048), (16, 32, 32)])
def test_hgravs01_low_rank_two_stage(ctx, oracle, rows, rank, cols):
    """y = L (R x) through hk_gemv_lowrank vs hgravs01_two_stage_matvec_f32
    and the FP64 product of the decoded factors; the (16, 32, 32) case is the
    reference's two-stage test shape with the rank raised to the kernel's
    32-column granularity (deterministic_matrix factors and input)."""
    from hawking_amd.organs import HgravS01LowRank
    say("hgravs01", rows, rank, cols)
    if rows == 16:
        Lw = oracle.deterministic_matrix(rows, rank, 3)
        Rw = oracle.deterministic_matrix(rank, cols, 5)
        x = oracle.deterministic_input(cols)
    else:
        Lw = oracle.normal(oracle.stream_key(U.SEED, 0xE1 + rank), rows * rank, 0.05).reshape(rows, rank)
        Rw = oracle.normal(oracle.stream_key(U.SEED, 0xE2 + rank), rank * cols, 0.02).reshape(rank, cols)
        x = oracle.normal(oracle.stream_key(U.SEED, 0xE3 + rank), cols, 1.0)
    left, (ls, lc) = _u3(ctx, oracle, Lw)
    right, (rs, rc) = _u3(ctx, oracle, Rw)
    lr = HgravS01LowRank(left, right)
    y = lr.matvec(x)
    ref = oracle.hgravs01_matvec((ls, lc), (rs, rc), rows, rank, cols, x, 3, 64)
    Ld = oracle.uniform_decode(ls, lc, rows, rank, 3, 64).astype(np.float64)
    Rd = oracle.uniform_decode(rs, rc, rank, cols, 3, 64).astype(np.float64)
    y64 = Ld @ (Rd @ x.astype(np.float64))
    assert oracle.relative_l2(y, ref) < TOL
    assert oracle.relative_l2(y, y64) < TOL


@pytest.mark.parametrize("shape", [(13, 96), (2048, 160)])
def test_synthetic_u3_factor_matches_oracle_pack(ctx, oracle, shape):
    """The device generator + 3-bit packer equals the oracle packing the
    oracle's draws (the bench's synthetic HGRAVS01 factors)."""
    from hawking_amd._lib import HK_U3
    from hawking_amd.organs import SyntheticOrgan
    rows, cols = shape
    key = oracle.stream_key(U.SEED, 0xD5 + rows)
    say("synthetic u3", shape)
    o = SyntheticOrgan(ctx, HK_U3, rows, cols, key, 0, group=64, sigma=0.05)
    s, c = oracle.uniform_pack(oracle.normal(key, rows * cols, 0.05), rows, cols, 3, 64)
    assert np.array_equal(o.decode(), oracle.uniform_decode(s, c, rows, cols, 3, 64))


def test_u3_and_lowrank_reject_bad_geometry(ctx, oracle):
    from hawking_amd._lib import HK_E_GEOMETRY, HawkingError
    from hawking_amd.organs import HgravS01LowRank, UniformFactor3
    s, c = oracle.uniform_pack(np.ones((16, 8), np.float32), 16, 8, 3, 64)
    with pytest.raises(HawkingError) as e:        # rank 8: not a multiple of 32 columns
        UniformFactor3(ctx, s, c, 16, 8)
    assert e.value.code == HK_E_GEOMETRY
    s, c = oracle.uniform_pack(np.ones((1, 7200), np.float32), 1, 7200, 3, 64)
    with pytest.raises(HawkingError) as e:        # past the 3-bit x image's 7168 columns (64 KB of LDS)
        UniformFactor3(ctx, s, c, 1, 7200)
    assert e.value.code == HK_E_GEOMETRY
    a, _ = _u3(ctx, oracle, np.ones((16, 64), np.float32))
    b, _ = _u3(ctx, oracle, np.ones((32, 32), np.float32))
    with pytest.raises(ValueError):
        HgravS01LowRank(a, b)
    mid, xd, yd = ctx.empty(64), ctx.empty(32), ctx.empty(16)
    with pytest.raises(HawkingError) as e:
        ctx.call("hk_gemv_lowrank", a.h, b.h, xd.ptr, mid.ptr, yd.ptr, ctx.stream)
    assert e.value.code == HK_E_GEOMETRY


@pytest.mark.parametrize("group,shape", [(64, (96, 1024)), (128, (7, 256)), (32, (1, 7168))])
def test_q4_other_groups_and_ragged_rows(ctx, oracle, group, shape):
    rows, cols = shape
    rng = np.random.default_rng(rows * cols + group)
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    say("q4", group, shape)
    organ, (s, c) = _q4(ctx, oracle, w, group)
    assert np.array_equal(organ.gather_row(rows - 1), oracle.q4_decode(s, c, rows, cols, group)[rows - 1])
    assert oracle.relative_l2(organ.matvec(x), oracle.q4_matvec_f64(s, c, rows, cols, group, x)) < TOL


def test_reference_deterministic_inputs(ctx, oracle):
    # deterministic_matrix(512, 2048, 1) / deterministic_input(2048): the inputs of the
    # reference's organ benchmark (examples/ascension_qwen80_matvec_geometry_sweep.rs).
    w = oracle.deterministic_matrix(512, 2048, 1)
    x = oracle.deterministic_input(2048)
    say("reference deterministic inputs")
    organ, (s, g) = _bin(ctx, oracle, w)
    assert oracle.relative_l2(organ.matvec(x), oracle.bin_matvec(s, g, 512, 2048, x)) < TOL
    organ, (s, c) = _q4(ctx, oracle, w, 64)
    assert oracle.relative_l2(organ.matvec(x), oracle.q4_matvec(s, c, 512, 2048, 64, x)) < TOL


def test_gemv_batch_matches_single(ctx, oracle):
    from hawking_amd.organs import gemv_batch
    rng = np.random.default_rng(21)
    n, rows, cols = 6, 512, 2048
    organs, refs = [], []
    xs = rng.standard_normal((n, cols)).astype(np.float32)
    for i in range(n):
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        o, (s, g) = _bin(ctx, oracle, w)
        organs.append(o)
        refs.append(oracle.bin_matvec(s, g, rows, cols, xs[i]))
    say("gemv_batch", n)
    xd = ctx.to_device(xs)
    yd = ctx.empty((n, rows))
    gemv_batch(ctx, organs, xd, cols, yd, rows)
    y = yd.download()
    for i in range(n):
        assert oracle.relative_l2(y[i], refs[i]) < TOL


def test_zero_input_gives_exact_zero(ctx, oracle):
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    organ, _ = _q4(ctx, oracle, w, 32)
    assert np.all(organ.matvec(np.zeros(512, np.float32)) == 0.0)


def test_upload_validation_errors(ctx, oracle):
    from hawking_amd._lib import HK_E_GEOMETRY, HK_E_NONFINITE, HK_E_UNSUPPORTED, HawkingError
    from hawking_amd.organs import BinaryGroupPacked, Qwen80Q4PackedTensor
    s, c = oracle.q4_pack(np.ones((4, 96), np.float32), 32)
    with pytest.raises(HawkingError) as e:
        Qwen80Q4PackedTensor(ctx, s[: 4 * 96 // 48], c, 4, 96, 48)
    assert e.value.code == HK_E_UNSUPPORTED
    bad = s.copy()
    bad[3] = 0x7C00                               # +inf scale
    with pytest.raises(HawkingError) as e:
        Qwen80Q4PackedTensor(ctx, bad, c, 4, 96, 32)
    assert e.value.code == HK_E_NONFINITE
    with pytest.raises(HawkingError) as e:
        BinaryGroupPacked(ctx, np.zeros(3, np.uint16), np.zeros(4 * 96 // 8, np.uint8), 4, 96)
    assert e.value.code == HK_E_GEOMETRY


def test_device_mixed_packer_bit_exact(ctx, oracle):
    """hk_pack_mixed (per-group selector over f32 weights) is bit-exact with
    the oracle's mixed pack, edge groups included, and its output uploads as
    an organ that decodes bit-exactly."""
    from hawking_amd import organs
    rng = np.random.default_rng(12)
    rows, cols = 64, 1024
    w = _edge_weights(rng, rows, cols)
    w[5, :64] = np.linspace(-1.5, 1.5, 64, dtype=np.float32)     # Q2 ties
    v0 = np.float32(2.0**-14 * (1 + 2.0**-11))                    # binary double rounding
    w[6, :128] = v0
    groups = rows * cols // 128
    for label, sel in (("coins", oracle.mixed_coins(oracle.stream_key(U.SEED, 0x31A), groups)),
                       ("all binary", np.ones(groups, np.uint8)), ("all q2", np.zeros(groups, np.uint8))):
        say("pack_mixed", label)
        tags, bs, bg, qs, qc = organs.pack_mixed_device(ctx, ctx.to_device(w), rows, cols, sel)
        m = oracle.mixed_pack(w, sel)
        nb, nq = m.n_bin, m.n_q2
        assert np.array_equal(tags.download(), m.tags)
        assert np.array_equal(bs.download()[:nb], m.bin_scales) and np.array_equal(bg.download()[:16 * nb], m.bin_signs)
        assert np.array_equal(qs.download()[:2 * nq], m.q2_scales) and np.array_equal(qc.download()[:32 * nq], m.q2_codes)
        o = organs.MixedPackedTensor(ctx, rows, cols, tags.download(), bs.download()[:nb], bg.download()[:16 * nb],
                                     qs.download()[:2 * nq], qc.download()[:32 * nq])
        assert np.array_equal(o.decode().view(np.uint32), oracle.mixed_decode(m).view(np.uint32))


def test_device_mixed_packer_capacity_and_rejects(ctx):
    from hawking_amd._lib import HK_E_INVALID_ARG, HK_E_NONFINITE, HawkingError
    rows, cols = 8, 256
    w = np.zeros((rows, cols), np.float32)
    sel = np.ones(rows * cols // 128, np.uint8)
    d = ctx.to_device(w)
    tags = ctx.empty(2, np.uint8)
    small = ctx.empty(64, np.uint8)
    n = C_uint32()
    with pytest.raises(HawkingError) as e:   # 16 binary groups, room for 4
        ctx.call("hk_pack_mixed", d.ptr, rows, cols, ctx.to_device(sel).ptr, tags.ptr, small.ptr, small.ptr, 4,
                 small.ptr, small.ptr, 0, n, ctx.stream)
    assert e.value.code == HK_E_INVALID_ARG
    w[3, 7] = np.inf
    from hawking_amd import organs
    with pytest.raises(HawkingError) as e:
        organs.pack_mixed_device(ctx, ctx.to_device(w), rows, cols, sel)
    assert e.value.code == HK_E_NONFINITE


def C_uint32():
    import ctypes
    return ctypes.byref(ctypes.c_uint32())


def test_gguf_q4_0_blocks_decode_bit_exact(ctx, oracle):
    """hk_organ_from_q4_0: GGUF Q4_0 AoS blocks (dequant_q4_0, quant.rs:473-498)
    bound as a Q4 group-32 organ decode bit for bit to the oracle's
    dequant_q4_0, and its matvec is within tolerance of the FP64 product."""
    from hawking_amd.containers import organ_from_q4_0
    rng = np.random.default_rng(40)
    rows, cols = 96, 2048
    nb = rows * cols // 32
    blocks = np.zeros((nb, 18), np.uint8)
    d = (rng.standard_normal(nb) * 0.003).astype(np.float16)
    d[0], d[1], d[2] = 0.0, np.float16(6.1e-5), np.float16(-0.25)   # zero, subnormal, negative scale
    blocks[:, :2] = d.view(np.uint8).reshape(nb, 2)
    blocks[:, 2:] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    blocks[3, 2:] = 0x0F      # low nibbles 15, high nibbles 0
    say("gguf q4_0", rows, cols)
    o = organ_from_q4_0(ctx, blocks, rows, cols)
    want = oracle.q4_0_dequant(blocks, rows * cols).reshape(rows, cols)
    assert np.array_equal(o.decode().view(np.uint32), want.view(np.uint32))
    x = rng.standard_normal(cols).astype(np.float32)
    y = o.matvec(x)
    assert oracle.relative_l2(y, want.astype(np.float64) @ x.astype(np.float64)) < TOL


def test_gguf_q4_0_rejects_bad_blocks(ctx):
    from hawking_amd._lib import HK_E_GEOMETRY, HK_E_NONFINITE, HawkingError
    from hawking_amd.containers import organ_from_q4_0
    blocks = np.zeros((8, 18), np.uint8)
    with pytest.raises(HawkingError) as e:
        organ_from_q4_0(ctx, blocks[:7], 4, 64)
    assert e.value.code == HK_E_GEOMETRY
    blocks[5, :2] = np.array([np.float16(np.inf)]).view(np.uint8)
    with pytest.raises(HawkingError) as e:
        organ_from_q4_0(ctx, blocks, 4, 64)
    assert e.value.code == HK_E_NONFINITE
