"""Pin the CPU oracle's packed formats against what the mathematics fixes.

The reference holds no fixture files for these organs (its organ parity lives
in examples that compare a GPU kernel with an in-process CPU oracle), so the
oracle is pinned here by: the IEEE binary16 / roundTiesToEven definitions
(numpy's independent implementations), hand-computed known answers, decode
closed forms, quantisation-error bounds, and brute-force f64 matvecs over the
decoded weights.  Each known answer is chosen so that a plausible slip
(nibble order, bit order, sign convention, rounding mode, a single instead of
a double rounding) fails it.
"""
import numpy as np
import pytest

# ---------------------------------------------------------------- IEEE helpers

def test_f16_to_f32_matches_numpy_on_every_bit_pattern(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref))


def test_f32_to_f16_round_to_nearest_even(oracle):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(0.02),
        rng.standard_normal(2000).astype(np.float32) * np.float32(1e-5),   # f16 subnormals
        rng.standard_normal(1000).astype(np.float32) * np.float32(3e4),    # near overflow
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, 2.0**-24, 2.0**-25,
                  1.5 * 2.0**-25, 2.0**-26, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11], np.float32),
    ])
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, ref)


def test_rint_ties_even(oracle):
    cases = {0.5: 0.0, 1.5: 2.0, 2.5: 2.0, -0.5: -0.0, -1.5: -2.0, -2.5: -2.0,
             0.49999997: 0.0, 7.5: 8.0, -8.5: -8.0, 3.2: 3.0, -3.7: -4.0}
    for v, want in cases.items():
        assert oracle.rint_ties_even(v) == want, v
    rng = np.random.default_rng(2)
    vals = (rng.standard_normal(5000) * 10).astype(np.float32)
    vals[::7] = np.round(vals[::7]) + np.float32(0.5)
    got = np.array([oracle.rint_ties_even(float(v)) for v in vals], np.float32)
    assert np.array_equal(got, np.rint(vals))


# ---------------------------------------------------------------- reference generators

def test_deterministic_generators_known_values(oracle):
    m = oracle.deterministic_matrix(2, 3, 1)
    # i=0: phase=f32(1) -> (1 % 251 - 125)/251
    assert m[0, 0] == np.float32(-124.0) / np.float32(251.0)
    # i=1: 1103515245 + 1 = 1103515246 -> f32 1103515264 -> fmod 251
    phase = np.float32(1103515246)
    assert m[0, 1] == (np.fmod(phase, np.float32(251)) - np.float32(125)) / np.float32(251)
    x = oracle.deterministic_input(20)
    assert x[0] == np.sin(np.float32(-0.5))
    assert x[17] == x[0] and x[18] == x[1]


# ---------------------------------------------------------------- Q4 uniform

def test_q4_known_answer_group32(oracle):
    g = np.zeros(32, np.float32)
    g[:12] = [7.0, -7.0, 0.5, 1.5, 2.5, -0.5, -1.5, 3.49, -2.5, 6.5, 0.0, -0.0]
    s, c = oracle.q4_pack(g.reshape(1, 32), 32)
    assert s.tolist() == [0x3C00]                       # f16(7/7) = 1.0
    q = [7, -7, 0, 2, 2, 0, -2, 3, -2, 6, 0, 0]            # rint ties-to-even
    codes = [v + 8 for v in q] + [8] * 20
    want = [codes[2 * i] | (codes[2 * i + 1] << 4) for i in range(16)]  # even index -> low nibble
    assert c.tolist() == want


def test_q4_zero_group_and_subnormal_clamp(oracle):
    z = np.zeros((1, 64), np.float32)
    s, c = oracle.q4_pack(z, 64)
    assert s.tolist() == [0] and set(c.tolist()) == {0x88}
    # max|w|/7 = 1.4*2^-24 rounds (f16 subnormal) down to 2^-24, so w/scale = -9.8
    # rounds to -10 and clamps to -8; +9.8 -> 10 -> clamps to 7.
    t = np.zeros((1, 32), np.float32)
    t[0, 0] = -9.8 * 2.0**-24
    t[0, 1] = 9.8 * 2.0**-24
    s, c = oracle.q4_pack(t, 32)
    assert s.tolist() == [1]
    assert c[0] == (0 | (15 << 4))


def test_q4_decode_closed_form(oracle):
    s = np.array([0x4000], np.uint16)                      # 2.0
    c = np.array([0xF0] + [0x00] * 15, np.uint8)           # local0 nibble 0, local1 nibble 15
    d = oracle.q4_decode(s, c, 1, 32, 32)[0]
    assert d[0] == -16.0 and d[1] == 14.0 and np.all(d[2:] == -16.0)


def test_q4_group_sizes(oracle):
    w = np.ones((4, 256), np.float32)
    for g in (32, 64, 128):
        s, c = oracle.q4_pack(w, g)
        assert s.size == 4 * 256 // g and c.size == 4 * 256 // 2
    for g in (0, 16, 96, 256, 512):
        with pytest.raises(oracle.OracleError):
            oracle.q4_pack(w, g)


@pytest.mark.parametrize("group", [32, 64, 128])
def test_q4_roundtrip_error_bound_and_matvec_vs_f64(oracle, group):
    rng = np.random.default_rng(group)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    s, c = oracle.q4_pack(w, group)
    d = oracle.q4_decode(s, c, 64, 512, group)
    scale = np.array([oracle.f16_to_f32(int(b)) for b in s], np.float32).repeat(group).reshape(64, 512)
    assert np.all(np.abs(d - w) <= scale * 0.5 * (1 + 2e-3) + 1e-12)
    # the per-group max element lands on +/-7 codes (up to the f16 rounding of max/7)
    codes = np.stack([c & 0xF, c >> 4], -1).reshape(-1).astype(np.int32) - 8
    assert codes.min() >= -8 and codes.max() <= 7
    x = rng.standard_normal(512).astype(np.float32)
    y = oracle.q4_matvec(s, c, 64, 512, group, x)
    y64 = d.astype(np.float64) @ x.astype(np.float64)
    assert oracle.relative_l2(y, y64) < 1e-6
    assert np.allclose(oracle.q4_matvec_f64(s, c, 64, 512, group, x), y64, rtol=1e-12, atol=1e-15)


def test_q4_matvec_rejects_nonfinite_input(oracle):
    s, c = oracle.q4_pack(np.ones((2, 32), np.float32), 32)
    x = np.ones(32, np.float32)
    x[3] = np.inf
    with pytest.raises(oracle.OracleError):
        oracle.q4_matvec(s, c, 2, 32, 32, x)


def test_q4_0_gguf_block_layout(oracle):
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[2:] = [j | ((15 - j) << 4) for j in range(16)]
    out = oracle.q4_0_dequant(blk, 32)
    assert out[:16].tolist() == [0.5 * (j - 8) for j in range(16)]      # low nibble -> j
    assert out[16:].tolist() == [0.5 * (7 - j) for j in range(16)]      # high nibble -> j+16


# ---------------------------------------------------------------- binary sign plane

def test_binary_known_answer_and_sign_of_negative_zero(oracle):
    g = np.concatenate([np.full(63, 1.0), [-0.0], np.full(64, -0.5)]).astype(np.float32)
    s, b = oracle.bin_pack(g.reshape(1, 128))
    # mean |w| = (63 + 0 + 32)/128 = 0.7421875, exactly representable in f16
    assert s.tolist() == [int(np.float16(0.7421875).view(np.uint16))]
    bits = np.unpackbits(b, bitorder="little")
    assert bits[:64].tolist() == [1] * 64                 # -0.0 >= 0 is true -> bit 1
    assert bits[64:].tolist() == [0] * 64
    d = oracle.bin_decode(s, b, 1, 128)[0]
    assert np.all(d[:64] == np.float32(0.7421875)) and np.all(d[64:] == -np.float32(0.7421875))


def test_binary_scale_is_double_rounded_f64_f32_f16(oracle):
    # f64 mean = v0 + 2^-44 with v0 = 2^-14 (1 + 2^-11): f32 drops the 2^-44,
    # leaving an exact f16 tie that rounds to even (0x0400).  Rounding the f64
    # mean straight to f16 would give 0x0401.
    v0 = np.float32(2.0**-14 * (1 + 2.0**-11))
    g = np.full(128, v0, np.float32)
    g[0] = np.nextafter(v0, np.float32(1))                # +1 f32 ulp = 2^-37
    mean64 = float(np.sum(g.astype(np.float64)) / 128)
    assert np.float16(mean64).view(np.uint16) == 0x0401
    s, _ = oracle.bin_pack(g.reshape(1, 128))
    assert s.tolist() == [0x0400]


def test_binary_reference_roundtrip_shape(oracle):
    # binary_group_roundtrip_signs_and_scales, q80_mixed_decode.rs:1433-1444
    w = oracle.deterministic_matrix(4, 256, 7)
    s, b = oracle.bin_pack(w)
    assert s.size == 4 * 2 and b.size == (4 * 256 + 7) // 8
    y = oracle.bin_matvec(s, b, 4, 256, oracle.deterministic_input(256))
    assert y.shape == (4,) and np.all(np.isfinite(y))


@pytest.mark.parametrize("shape", [(512, 2048), (2048, 512)])
def test_binary_matvec_vs_f64(oracle, shape):
    rows, cols = shape
    rng = np.random.default_rng(rows)
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    s, b = oracle.bin_pack(w)
    d = oracle.bin_decode(s, b, rows, cols)
    assert np.array_equal(np.signbit(d), w < 0)
    x = rng.standard_normal(cols).astype(np.float32)
    y = oracle.bin_matvec(s, b, rows, cols, x)
    y64 = d.astype(np.float64) @ x.astype(np.float64)
    assert oracle.relative_l2(y, y64) < 1e-5
    means = np.abs(w.astype(np.float64)).reshape(rows, cols // 128, 128).mean(-1)
    assert np.array_equal(s, means.astype(np.float32).astype(np.float16).view(np.uint16).reshape(-1))


# ---------------------------------------------------------------- Q2 stage

def test_q2_known_answer(oracle):
    g = np.zeros(64, np.float32)
    g[:10] = [1.5, -1.5, 0.0, -1.0, 1.0, 0.5, -0.5, 0.99, 1.01, -0.0]
    s, c = oracle.q2_pack(g)
    assert s.tolist() == [0x3C00]                       # f16(1.5/1.5) = 1.0
    # code = rint(w + 1.5) with ties to even, clipped to [0, 3]
    want = [3, 0, 2, 0, 2, 2, 1, 2, 3, 2] + [2] * 54
    got = [(c[e >> 2] >> (2 * (e & 3))) & 3 for e in range(64)]   # 2-bit LSB-first
    assert got == want
    d = oracle.q2_decode(s, c, 64)
    assert d[:4].tolist() == [1.5, -1.5, 0.5, -1.5]


def test_q2_zero_group_divides_by_one(oracle):
    s, c = oracle.q2_pack(np.zeros(64, np.float32))
    assert s.tolist() == [0] and set(c.tolist()) == {0b10101010}
    assert np.all(oracle.q2_decode(s, c, 64) == 0)


def test_q2_error_bound(oracle):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal(64 * 200) * 0.02).astype(np.float32)
    s, c = oracle.q2_pack(w)
    d = oracle.q2_decode(s, c, w.size)
    sc = np.array([oracle.f16_to_f32(int(b)) for b in s], np.float32).repeat(64)
    # levels are scale*{-1.5..1.5} spaced by scale; max |w| <= 1.5*scale (1+2^-11)
    assert np.all(np.abs(d - w) <= sc * 0.5 * (1 + 1e-3) + 1e-12)


# ---------------------------------------------------------------- mixed

def test_mixed_stream_layout(oracle):
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((2, 256)) * 0.02).astype(np.float32)
    sel = np.array([1, 0, 0, 1], np.uint8)   # flat groups: (r0,g0) bin, (r0,g1) q2, (r1,g0) q2, (r1,g1) bin
    m = oracle.mixed_pack(w, sel)
    assert m.tags.tolist() == [0b1001]
    assert m.n_bin == 2 and m.n_q2 == 2
    s0, b0 = oracle.bin_pack(w[0:1, :128])
    s3, b3 = oracle.bin_pack(w[1:2, 128:])
    assert m.bin_scales.tolist() == [s0[0], s3[0]]
    assert np.array_equal(m.bin_signs, np.concatenate([b0, b3]))
    qs1, qc1 = oracle.q2_pack(w[0, 128:])
    qs2, qc2 = oracle.q2_pack(w[1, :128])
    assert m.q2_scales.tolist() == qs1.tolist() + qs2.tolist()
    assert np.array_equal(m.q2_codes, np.concatenate([qc1, qc2]))
    d = oracle.mixed_decode(m)
    assert np.array_equal(d[0, :128], oracle.bin_decode(s0, b0, 1, 128)[0])
    assert np.array_equal(d[0, 128:], oracle.q2_decode(qs1, qc1, 128))


def test_mixed_matvec_vs_f64_and_density(oracle):
    rng = np.random.default_rng(11)
    rows, cols = 512, 2048
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    key = oracle.stream_key(0x48415752, 77)
    sel = oracle.mixed_coins(key, rows * cols // 128)
    assert abs(sel.mean() - 0.7) < 0.02
    m = oracle.mixed_pack(w, sel)
    bpw = 8 * m.nbytes() / (rows * cols)
    assert 1.40 < bpw < 1.52
    x = rng.standard_normal(cols).astype(np.float32)
    y = oracle.mixed_matvec(m, x)
    y64 = oracle.mixed_decode(m).astype(np.float64) @ x.astype(np.float64)
    assert oracle.relative_l2(y, y64) < 1e-5
    assert np.allclose(oracle.mixed_matvec_f64(m, x), y64, rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------- synthetic generator

def test_normal_generator_statistics_and_grid(oracle):
    key = oracle.stream_key(0x48415752, 1)
    z = oracle.normal(key, 200000, 1.0)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert np.all(np.abs(z) <= 6.0)
    assert np.array_equal(z * 131072, np.round(z * 131072))   # exact multiples of 2^-17
    w = oracle.normal(key, 1000, 0.02)
    assert np.array_equal(w, z[:1000] * np.float32(0.02))
    assert not np.array_equal(oracle.normal(oracle.stream_key(0x48415752, 2), 1000, 1.0), z[:1000])
