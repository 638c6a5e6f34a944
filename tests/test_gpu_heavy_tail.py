"""Heavy-tailed inputs on every organ kind: the engine's fixed-point x image
keeps each element to 24 bits of its own unit's max (one exponent per
zero-point unit of SXG columns), so one element of x orders of magnitude
above the rest does not coarsen the others.

Per row i, against the FP64 product of the decoded weights:
  |y_i - y64_i| <= sum_u max(2^-23 max_{j in u}|x_j|, 2^-121) sum_{j in u}|w_ij|   (x quantization)
                 + (n_units + 4) 2^-24 sum_j |w_ij x_j|                          (f32 combine and sums)
a worst-case bound; 2^-121 is the floor of the per-unit exponent cap (a
unit whose max is below 2^-98 is quantized to 2^-120).  An input scaled to
1e-30 throughout (every unit near that floor) checks it.  Whole vectors: rel-L2 <= 2e-5 against the FP64
product and the oracle's serial f32 path, and no worse than the serial f32
path itself: rel-L2(engine, FP64) <= 2 rel-L2(serial f32, FP64) + 2e-7 --
the check an engine with one exponent for the whole vector (every element
quantized to 2^-24 of max|x|: about 2e-6 on the spike inputs against the
serial path's 8e-7) fails.
"""
import sys

import numpy as np
import pytest

from tests import hk_testutil as U

pytestmark = pytest.mark.gpu
TOL = 2e-5
ROWS, COLS = 256, 2048


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    from hawking_amd.runtime import Context
    return Context(0)


def inputs(seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(COLS).astype(np.float32)
    spike = x.copy()
    spike[777] = np.float32(1e4 * np.median(np.abs(x)))
    zeros = x.copy()
    zeros[rng.random(COLS) < 0.75] = 0.0
    zeros[5] = np.float32(-1e4)
    t2 = rng.standard_t(2, COLS).astype(np.float32)
    tiny = (x * np.float32(1e-30)).astype(np.float32)
    tiny1 = tiny.copy()
    tiny1[9] = np.float32(3.0)
    return {"spike 1e4x median": spike, "75% zeros + spike": zeros, "student-t(2)": t2,
            "1e-30 scale + one O(1)": tiny1, "1e-30 scale": tiny}


def organ_and_weights(ctx, oracle, kind, seed):
    from hawking_amd import organs
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((ROWS, COLS)) * 0.02).astype(np.float32)
    if kind == "q4":
        s, c = oracle.q4_pack(w, 32)
        return organs.Qwen80Q4PackedTensor(ctx, s, c, ROWS, COLS, 32), oracle.q4_decode(s, c, ROWS, COLS, 32), 32, \
            lambda x: oracle.q4_matvec(s, c, ROWS, COLS, 32, x)
    if kind == "binary":
        s, g = oracle.bin_pack(w)
        return organs.BinaryGroupPacked(ctx, s, g, ROWS, COLS), oracle.bin_decode(s, g, ROWS, COLS), 128, \
            lambda x: oracle.bin_matvec(s, g, ROWS, COLS, x)
    if kind == "mixed":
        m = oracle.mixed_pack(w, oracle.mixed_coins(oracle.stream_key(U.SEED, 0x7A11), ROWS * COLS // 128))
        o = organs.MixedPackedTensor(ctx, ROWS, COLS, m.tags, m.bin_scales, m.bin_signs, m.q2_scales, m.q2_codes)
        return o, oracle.mixed_decode(m), 64, lambda x: oracle.mixed_matvec(m, x)
    if kind == "q8":
        s, c = oracle.uniform_pack(w, ROWS, COLS, 8, 64)
        return organs.UniformFactorPacked(ctx, s, c, ROWS, COLS), oracle.uniform_decode(s, c, ROWS, COLS, 8, 64), 16, \
            lambda x: oracle.uniform_matvec(s, c, ROWS, COLS, x, 8, 64)
    s, c = oracle.uniform_pack(w, ROWS, COLS, 3, 64)
    return organs.UniformFactor3(ctx, s, c, ROWS, COLS), oracle.uniform_decode(s, c, ROWS, COLS, 3, 64), 32, \
        lambda x: oracle.uniform_matvec(s, c, ROWS, COLS, x, 3, 64)


def row_bound(W64, x, unit):
    ax = np.abs(x.astype(np.float64))
    umax = ax.reshape(-1, unit).max(axis=1)                      # per-unit max |x|
    aw = np.abs(W64)
    ustep = np.maximum(umax * 2.0 ** -23, 2.0 ** -121)
    quant = (aw.reshape(ROWS, -1, unit).sum(axis=2) * ustep[None, :]).sum(axis=1)
    acc = (COLS // unit + 4) * 2.0 ** -24 * (aw @ ax)
    return quant + acc


@pytest.mark.parametrize("kind", ["q4", "binary", "mixed", "q8", "u3"])
def test_heavy_tailed_x_per_row_bound(ctx, oracle, kind):
    organ, Wd, unit, serial = organ_and_weights(ctx, oracle, kind, 400 + len(kind))
    W64 = np.asarray(Wd, np.float64).reshape(ROWS, COLS)
    for label, x in inputs(len(kind)).items():
        say("heavy tail", kind, label)
        y = organ.matvec(x).astype(np.float64)
        y64 = W64 @ x.astype(np.float64)
        err = np.abs(y - y64)
        bound = row_bound(W64, x, unit)
        worst = int(np.argmax(err / bound))
        assert np.all(err <= bound), (kind, label, worst, err[worst], bound[worst])
        ys = serial(x)
        assert oracle.relative_l2(y, y64) < TOL, (kind, label)
        assert oracle.relative_l2(y, ys) < TOL, (kind, label)
        assert oracle.relative_l2(y, y64) <= 2.0 * oracle.relative_l2(ys, y64) + 2e-7, (kind, label)


def test_heavy_tailed_x_low_rank_and_rice(ctx, oracle):
    """The two-stage HGRAVS01 organ (mid = R x goes through a second x image)
    and the HGRAVR02 base + residual, on the same inputs: rel-L2 vs FP64."""
    from hawking_amd import organs
    rng = np.random.default_rng(77)
    Lw = (rng.standard_normal((ROWS, 160)) * 0.05).astype(np.float32)
    Rw = (rng.standard_normal((160, COLS)) * 0.02).astype(np.float32)
    ls, lc = oracle.uniform_pack(Lw, ROWS, 160, 3, 64)
    rs, rc = oracle.uniform_pack(Rw, 160, COLS, 3, 64)
    lr = organs.HgravS01LowRank(organs.UniformFactor3(ctx, ls, lc, ROWS, 160), organs.UniformFactor3(ctx, rs, rc, 160, COLS))
    Ld = oracle.uniform_decode(ls, lc, ROWS, 160, 3, 64).astype(np.float64).reshape(ROWS, 160)
    Rd = oracle.uniform_decode(rs, rc, 160, COLS, 3, 64).astype(np.float64).reshape(160, COLS)
    w = (rng.standard_normal((ROWS, COLS)) * 0.02).astype(np.float32)
    p = oracle.rice_q1_pack(w, ROWS, COLS, 0.02)
    rice = organs.RiceQ1Packed(ctx, p.rows, p.cols, p.bin_scales, p.bin_signs, p.first, p.rice_k, p.rice, p.count,
                               p.res_scale, p.res_signs)
    for label, x in inputs(5).items():
        say("heavy tail low-rank / rice", label)
        y = organs.hgravs01_two_stage_matvec_f32(lr, x)
        assert oracle.relative_l2(y, Ld @ (Rd @ x.astype(np.float64))) < TOL, label
        yr = organs.binary_rice_q1_matvec_f32(rice, x)
        assert oracle.relative_l2(yr, oracle.rice_q1_matvec_f64(p, x)) < TOL, label
