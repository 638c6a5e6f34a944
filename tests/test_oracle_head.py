"""The oracle's terminal head (terminal_greedy,
qwen80_mixed_hybrid_decode.rs:3754-3790): the greedy pick's tie, NaN, mask
and error rules by known answers, and the whole head against an f64 argmax
of the decoded lm_head.  CPU only."""
import numpy as np
import pytest


def test_greedy_pick_rules(oracle):
    f = np.float32
    assert oracle.argmax_greedy(np.array([1, 3, 3, 2], f)) == 1                 # first maximum
    assert oracle.argmax_greedy(np.array([np.nan, -1, np.nan, -2], f)) == 1     # NaN never wins
    assert oracle.argmax_greedy(np.array([0.0, -0.0, 0.0], f)) == 0             # -0 == +0: a tie
    assert oracle.argmax_greedy(np.array([-0.0, 0.0], f)) == 0
    assert oracle.argmax_greedy(np.array([-5, -4, 9e9], f), n_valid=2) == 1     # masked tail ignored
    for bad in ([np.nan, np.nan], [-np.inf, -np.inf], [1.0, np.inf], []):
        with pytest.raises(oracle.OracleError):
            oracle.argmax_greedy(np.array(bad, f))


def test_head_against_f64(oracle):
    rng = np.random.default_rng(1)
    hidden_n, vocab, n_valid = 256, 640, 600
    h = rng.standard_normal(hidden_n).astype(np.float32)
    nw = (rng.standard_normal(hidden_n) * 0.02).astype(np.float32)
    w = (rng.standard_normal((vocab, hidden_n)) * 0.05).astype(np.float32)
    s, c = oracle.uniform_pack(w, vocab, hidden_n, 8, 64)
    tok, logits = oracle.terminal_greedy(h, nw, s, c, vocab, n_valid)
    xn = oracle.rmsnorm_1p(h, nw, 1e-6).astype(np.float64)
    ref = oracle.uniform_decode(s, c, vocab, hidden_n, 8, 64).astype(np.float64) @ xn
    assert np.linalg.norm(logits - ref) / np.linalg.norm(ref) < 1e-6
    top2 = np.sort(ref[:n_valid])[-2:]
    assert top2[1] - top2[0] > 1e-4 * np.abs(ref).max()      # the pick is well separated here
    assert tok == int(np.argmax(ref[:n_valid]))
