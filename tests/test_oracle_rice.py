"""The oracle's HGRAVR02 codec (binary base + Rice-coded 1-bit residual,
pack_binary_rice_q1 / pack_rice / unpack_rice / expand_rice_indices /
rice_q1_row_ptr / binary_rice_q1_matvec_f32, q80_mixed_decode.rs:260-527)
pinned by hand-derived known answers: the Rice bit order and layout, the
choice of k (first on ties), the residual's definition, the top-count
selection with its lower-index tie rule, the sign bits and the f16 RMS scale.
CPU only."""
import numpy as np
import pytest


def test_rice_bitstream_known_answers(oracle):
    # k = 1: 5 -> 1 1 0 | 1;  0 -> 0 | 0;  3 -> 1 0 | 1  (LSB-first bytes)
    assert oracle.rice_pack([5, 0, 3], 1).tolist() == [0x4B, 0x01]
    # k = 0: 2 -> 1 1 0;  1 -> 1 0
    assert oracle.rice_pack([2, 1], 0).tolist() == [0x0B]
    assert oracle.rice_unpack([0x4B, 0x01], 3, 1).tolist() == [5, 0, 3]
    with pytest.raises(oracle.OracleError):        # the stream ends inside the third value
        oracle.rice_unpack([0x4B], 3, 1)


def test_best_rice_k_first_minimum(oracle):
    # ten 100s: bits(6) = 10 + 70 = bits(7) = 0 + 80 < bits(5) = 90 -> the first, 6
    assert oracle.best_rice_k([100] * 10) == 6
    assert oracle.best_rice_k([0] * 5) == 0
    assert oracle.best_rice_k([]) == 0
    # the reference's cost over every k, by brute force, for random values
    rng = np.random.default_rng(4)
    v = rng.integers(1, 3000, 200).astype(np.uint32)
    costs = [int((v >> k).sum()) + v.size * (1 + k) for k in range(16)]
    assert oracle.best_rice_k(v) == int(np.argmin(costs))


@pytest.mark.parametrize("k", range(16))
def test_rice_roundtrip_every_k(oracle, k):
    rng = np.random.default_rng(k)
    v = rng.integers(0, 1 << min(k + 3, 20), 300).astype(np.uint32)
    assert np.array_equal(oracle.rice_unpack(oracle.rice_pack(v, k), v.size, k), v)


def test_expand_and_row_ptr(oracle):
    rice = oracle.rice_pack([5, 0, 3], 1)
    assert oracle.rice_expand(10, rice, 1, 4).tolist() == [10, 15, 15, 18]
    assert oracle.rice_expand(7, np.zeros(0, np.uint8), 0, 1).tolist() == [7]
    with pytest.raises(oracle.OracleError):        # 2^32 - 2 + 5 exceeds u32
        oracle.rice_expand(2 ** 32 - 2, oracle.rice_pack([5], 0), 0, 2)
    assert oracle.rice_row_ptr([0, 5, 130, 131, 700], 6, 128).tolist() == [0, 2, 4, 4, 4, 4, 5]
    with pytest.raises(oracle.OracleError):
        oracle.rice_row_ptr([0, 768], 6, 128)


def test_pack_known_answer(oracle):
    # one row of 1s with 3.0 at 5 and 77 and -2.0 at 9: binary scale 133/128
    # (exact in f16), residuals 1.9609375 (x2), -0.9609375, -0.0390625 (x125)
    w = np.ones(128, np.float32)
    w[5], w[9], w[77] = 3.0, -2.0, 3.0
    p = oracle.rice_q1_pack(w, 1, 128, 0.02)            # count = ceil(2.56) = 3
    assert p.bin_scales.tolist() == [0x3C28]
    assert p.indices.tolist() == [5, 9, 77]
    assert p.res_signs.tolist() == [0b101]
    # sqrt((2 * 1.9609375^2 + 0.9609375^2) / 3) = 1.69449... -> f16 1735/1024
    assert p.res_scale == 0x3EC7
    # diffs [4, 68]: k = 4 (ties with 5, first wins); 4 -> 0|0010, 68 -> 11110|0010
    assert (p.first, p.rice_k, p.rice.tolist()) == (5, 4, [0xE8, 0x11])
    # ratio 0.005 -> one outlier: the |r| tie between 5 and 77 goes to the lower index
    p1 = oracle.rice_q1_pack(w, 1, 128, 0.005)
    assert (p1.indices.tolist(), p1.first, p1.rice.size) == ([5], 5, 0)
    with pytest.raises(oracle.OracleError):
        oracle.rice_q1_pack(w, 1, 128, 0.2)               # ratio outside (0, 0.1]


def test_selection_matches_a_numpy_ranking(oracle):
    """Top-count |residual| with ties to the lower index, checked against
    numpy's lexsort of the residual computed from the oracle's decoded base,
    on data with many exact ties (weights on a coarse grid)."""
    rng = np.random.default_rng(21)
    rows, cols = 12, 256
    w = (rng.integers(-8, 9, (rows, cols)) / 8.0).astype(np.float32)
    p = oracle.rice_q1_pack(w, rows, cols, 0.03)
    base = oracle.bin_decode(p.bin_scales, p.bin_signs, rows, cols)
    r = (w - base).reshape(-1)
    order = np.lexsort((np.arange(r.size), -np.abs(r)))
    assert np.array_equal(p.indices, np.sort(order[:p.count]).astype(np.uint32))
    assert np.array_equal(np.unpackbits(p.res_signs, bitorder="little")[:p.count], (r[p.indices] >= 0))
    assert np.array_equal(oracle.rice_expand(p.first, p.rice, p.rice_k, p.count), p.indices)


def test_reference_rice_cases(oracle):
    # rice_q1_indices_roundtrip and rice_q1_fused_correction_does_not_form_dense_w
    # (q80_mixed_decode.rs:1447-1496): 8 x 128 deterministic_matrix(seed 11) at 2%
    rows, cols = 8, 128
    w = oracle.deterministic_matrix(rows, cols, 11)
    p = oracle.rice_q1_pack(w, rows, cols, 0.02)
    assert p.count == 21
    assert np.array_equal(oracle.rice_expand(p.first, p.rice, p.rice_k, p.count), p.indices)
    x = oracle.deterministic_input(cols)
    y = oracle.rice_q1_matvec(p, x)
    assert np.all(np.isfinite(y))
    base = oracle.bin_matvec(p.bin_scales, p.bin_signs, rows, cols, x)
    assert np.array_equal(oracle.rice_q1_apply(p, x, base), y)
    # against the f64 product of the decoded base plus the signed residual
    dense = oracle.bin_decode(p.bin_scales, p.bin_signs, rows, cols).astype(np.float64).reshape(-1)
    s = oracle.f16_to_f32(p.res_scale)
    bits = np.unpackbits(p.res_signs, bitorder="little")[:p.count]
    dense[p.indices] += np.where(bits == 1, s, -s)
    ref = dense.reshape(rows, cols) @ x.astype(np.float64)
    assert np.allclose(oracle.rice_q1_matvec_f64(p, x), ref, rtol=1e-12, atol=1e-12)
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-6


def test_rice_pack_is_thread_safe(oracle):
    """Packs running on several threads at once (the GPU parity tests
    generate experts on a thread pool) give the serial packs' bytes."""
    import concurrent.futures as cf
    ws = [oracle.normal(oracle.stream_key(0x7E5, i), 64 * 512, 0.02).reshape(64, 512) for i in range(16)]
    serial = [oracle.rice_q1_pack(w, 64, 512, 0.02) for w in ws]
    with cf.ThreadPoolExecutor(max_workers=8) as pool:
        for _ in range(3):
            par = list(pool.map(lambda w: oracle.rice_q1_pack(w, 64, 512, 0.02), ws))
            for a, b in zip(serial, par):
                assert np.array_equal(a.indices, b.indices) and np.array_equal(a.rice, b.rice)
                assert np.array_equal(a.res_signs, b.res_signs) and a.res_scale == b.res_scale
