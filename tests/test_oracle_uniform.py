"""The oracle's uniform factor codec (HGRAVU01 q8 G64, HGRAVS01 3-bit
factors; pack_uniform_factor / uniform_factor_value / uniform_factor_matvec_f32
/ hgravs01_two_stage_matvec_f32, q80_mixed_decode.rs:529-629) pinned by known
answers: the rounding mode, the quantizer's divisor, the f16 scale rounding,
the LSB-first bit order, group padding, and matvec against an f64 dot of the
decoded weights.  CPU only."""
import numpy as np
import pytest

D = 1.0 + 2.0 ** -11   # exact in f32; f16 rounds it (a tie) to even = 1.0


def test_q8_known_answer_rounding_divisor_and_scale(oracle):
    # max = 127 * D: the f32 scale is D, its f16 is 1.0 (round half to even).
    # 62.5 * D / D = 62.5 exactly -> rounds half AWAY from zero to 63 (code 190);
    # 62.5 / D = 62.47 -> 62 (code 189) -- 63 if the f16 scale were the divisor.
    g = np.zeros(64, np.float32)
    g[0], g[1], g[2], g[3] = 127 * D, 62.5 * D, 62.5, -62.5 * D
    s, c = oracle.uniform_pack(g, 1, 64, 8, 64)
    assert s.tolist() == [0x3C00]
    assert c.tolist() == [254, 190, 189, 64] + [127] * 60
    assert oracle.uniform_decode(s, c, 1, 64, 8, 64)[0, :5].tolist() == [127.0, 63.0, 62.0, -63.0, 0.0]


def test_three_bit_codes_are_lsb_first(oracle):
    # bound 3, scale 1: values -3..3 -> codes 0..6; hand-packed bitstream
    w = np.array([-3, -2, -1, 0, 1, 2, 3, 0], np.float32)
    s, c = oracle.uniform_pack(w, 1, 8, 3, 8)
    assert s.tolist() == [0x3C00]
    assert c.tolist() == [0x88, 0xC6, 0x7A]
    assert oracle.uniform_decode(s, c, 1, 8, 3, 8)[0].tolist() == w.tolist()


def test_padding_zero_groups_and_byte_count(oracle):
    rng = np.random.default_rng(1)
    w = rng.standard_normal((3, 5)).astype(np.float32)
    w[0, :] = 0.0
    s, c = oracle.uniform_pack(w, 3, 5, 8, 8)       # 15 elements -> 2 groups, 16 codes
    assert s.size == 2 and c.size == 16
    assert c[15] == 127                              # the padding code is the zero level
    z = np.zeros(64, np.float32)
    s0, c0 = oracle.uniform_pack(z, 1, 64, 8, 64)
    assert s0.tolist() == [0] and set(c0.tolist()) == {127}
    assert not np.any(oracle.uniform_decode(s0, c0, 1, 64, 8, 64))
    with pytest.raises(oracle.OracleError):
        oracle.uniform_pack(np.array([np.nan] + [0.0] * 63, np.float32), 1, 64, 8, 64)


@pytest.mark.parametrize("bits", [8, 3])
def test_roundtrip_error_bound(oracle, bits):
    rng = np.random.default_rng(bits)
    rows, cols = 16, 256
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    s, c = oracle.uniform_pack(w, rows, cols, bits, 64)
    dec = oracle.uniform_decode(s, c, rows, cols, bits, 64).reshape(-1)
    bound = (1 << (bits - 1)) - 1
    sf = np.array([oracle.f16_to_f32(int(v)) for v in s], np.float32)
    g = np.abs(w.reshape(-1, 64)).max(axis=1) / np.float32(bound)     # the f32 scales
    err = np.abs(dec - w.reshape(-1)).reshape(-1, 64)
    assert np.all(err <= (0.5 * g + bound * np.abs(sf - g))[:, None] * (1 + 1e-6) + 1e-12)


def test_matvec_is_the_serial_dot_of_the_decoded_weights(oracle):
    rng = np.random.default_rng(7)
    rows, cols = 33, 448
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    s, c = oracle.uniform_pack(w, rows, cols, 8, 64)
    dec = oracle.uniform_decode(s, c, rows, cols, 8, 64).astype(np.float64)
    y = oracle.uniform_matvec(s, c, rows, cols, x, 8, 64)
    y64 = oracle.uniform_matvec_f64(s, c, rows, cols, x, 8, 64)
    ref = dec @ x.astype(np.float64)
    assert np.allclose(y64, ref, rtol=1e-12, atol=1e-12)
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 2e-6


def test_hgravs01_two_stage_reference_case(oracle):
    # hgravs_two_stage_does_not_need_dense_w (q80_mixed_decode.rs:1462-1476)
    rows, cols, rank = 16, 32, 8
    L = oracle.deterministic_matrix(rows, rank, 3)
    R = oracle.deterministic_matrix(rank, cols, 5)
    left = oracle.uniform_pack(L, rows, rank, 3, 64)
    right = oracle.uniform_pack(R, rank, cols, 3, 64)
    x = oracle.deterministic_input(cols)
    y = oracle.hgravs01_matvec(left, right, rows, rank, cols, x, 3, 64)
    assert y.shape == (rows,) and np.all(np.isfinite(y))
    Ld = oracle.uniform_decode(*left, rows, rank, 3, 64).astype(np.float64)
    Rd = oracle.uniform_decode(*right, rank, cols, 3, 64).astype(np.float64)
    ref = Ld @ (Rd @ x.astype(np.float64))
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-6
