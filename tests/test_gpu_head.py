"""GPU parity of the device-side terminal head (hk_terminal_greedy) against
the oracle's terminal_greedy: logits within 2e-5 relative L2 of the serial
f32 path and the FP64 authority; the token equal to the oracle's when the
top two logits are separated (the margin rule), and exact on constructed
ties, masks and error cases."""
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


def _head(ctx, oracle, w, nw, n_valid):
    from hawking_amd.head import TerminalHead
    from hawking_amd.organs import UniformFactorPacked
    vocab, hidden_n = w.shape
    s, c = oracle.uniform_pack(w, vocab, hidden_n, 8, 64)
    return TerminalHead(ctx, nw, UniformFactorPacked(ctx, s, c, vocab, hidden_n), n_valid), (s, c)


def _inputs(oracle, vocab, hidden_n, tag):
    key = lambda k: oracle.stream_key(U.SEED, (0xF0 << 8) + k + vocab)
    h = oracle.normal(key(1), hidden_n, 1.0)
    nw = oracle.normal(key(2), hidden_n, 0.02)
    w = oracle.normal(key(3), vocab * hidden_n, 0.05).reshape(vocab, hidden_n)
    return h, nw, w


@pytest.mark.parametrize("vocab,hidden_n,n_valid", [(4096, 2048, 4000), (151936, 256, 151669), (640, 512, 640)])
def test_terminal_head_matches_oracle(ctx, oracle, vocab, hidden_n, n_valid):
    h, nw, w = _inputs(oracle, vocab, hidden_n, "n")
    say("terminal head", vocab, hidden_n, n_valid)
    head, (s, c) = _head(ctx, oracle, w, nw, n_valid)
    tok = head.greedy(h)
    ref_tok, ref_logits = oracle.terminal_greedy(h, nw, s, c, vocab, n_valid)
    logits = head.logits.download()
    xn = oracle.rmsnorm_1p(h, nw, 1e-6).astype(np.float64)
    ref64 = oracle.uniform_matvec_f64(s, c, vocab, hidden_n, xn, 8, 64)
    assert oracle.relative_l2(logits, ref_logits) < TOL
    assert oracle.relative_l2(logits, ref64) < TOL
    top2 = np.sort(ref64[:n_valid])[-2:]
    if top2[1] - top2[0] > 1e-4 * np.abs(ref64).max():
        assert tok == ref_tok
    # the device pick over the device logits follows the reference's rule exactly
    assert tok == oracle.argmax_greedy(logits, n_valid)


def test_terminal_head_tie_and_mask(ctx, oracle):
    """Two identical lm_head rows that dominate give identical logits on the
    device; the lower index wins.  A larger row past n_valid is never chosen."""
    vocab, hidden_n, n_valid = 1024, 512, 1000
    h, nw, w = _inputs(oracle, vocab, hidden_n, "t")
    xn = oracle.rmsnorm_1p(h, nw, 1e-6)
    strong = (0.05 * np.sign(xn)).astype(np.float32)
    w[[37, 900]] = strong
    w[1010] = 2.0 * strong                      # masked
    say("terminal head tie/mask")
    head, _ = _head(ctx, oracle, w, nw, n_valid)
    assert head.greedy(h) == 37
    lg = head.logits.download()
    assert lg[37] == lg[900] and lg[1010] > lg[37]


@pytest.mark.parametrize("value", [np.inf, np.nan])
def test_terminal_head_flags_nonfinite(ctx, oracle, value):
    """A non-finite hidden state (inf, or a NaN, which a plain max would
    drop) gives token -1 and HK_E_NONFINITE; the next good call recovers."""
    from hawking_amd._lib import HK_E_NONFINITE, HawkingError
    vocab, hidden_n = 256, 256
    h, nw, w = _inputs(oracle, vocab, hidden_n, "e")
    head, _ = _head(ctx, oracle, w, nw, vocab)
    bad = h.copy()
    bad[7] = value
    say("terminal head non-finite", value)
    with pytest.raises(HawkingError) as e:
        head.greedy(bad)
    assert e.value.code == HK_E_NONFINITE
    assert int(head.token.download()[0]) == -1
    assert head.greedy(h) == oracle.argmax_greedy(head.logits.download())   # recovers on good input


def test_two_heads_share_one_lm_head_on_two_streams(ctx, oracle):
    """The lm_head organ is read-only: two heads over one lm_head with their
    own workspaces run on two streams at once and each gets its own token."""
    from hawking_amd.head import TerminalHead
    from hawking_amd.organs import UniformFactorPacked
    vocab, hidden_n = 8192, 1024
    h1, nw, w = _inputs(oracle, vocab, hidden_n, "s")
    h2 = oracle.normal(oracle.stream_key(U.SEED, 0xF2F2), hidden_n, 1.0)
    s, c = oracle.uniform_pack(w, vocab, hidden_n, 8, 64)
    lm = UniformFactorPacked(ctx, s, c, vocab, hidden_n)
    a, b = TerminalHead(ctx, nw, lm), TerminalHead(ctx, nw, lm)
    sa, sb = ctx.new_stream(), ctx.new_stream()
    say("two heads, two streams")
    refs = [oracle.terminal_greedy(hh, nw, s, c, vocab, vocab) for hh in (h1, h2)]
    d1, d2 = ctx.to_device(h1), ctx.to_device(h2)
    ctx.synchronize()
    for _ in range(20):
        a.greedy_device(d1, stream=sa)
        b.greedy_device(d2, stream=sb)
    ctx.call("hk_stream_synchronize", sa)
    ctx.call("hk_stream_synchronize", sb)
    ta, tb = int(a.token.download()[0]), int(b.token.download()[0])
    assert ta == oracle.argmax_greedy(a.logits.download(), vocab)
    assert tb == oracle.argmax_greedy(b.logits.download(), vocab)
    for tok, head, (rtok, rlog) in ((ta, a, refs[0]), (tb, b, refs[1])):
        assert oracle.relative_l2(head.logits.download(), rlog) < TOL
        top2 = np.sort(rlog)[-2:]
        if top2[1] - top2[0] > 1e-4 * np.abs(rlog).max():
            assert tok == rtok
    assert a.pick.download().tolist() == [0, 0] and b.pick.download().tolist() == [0, 0]
    ctx.call("hk_stream_destroy", sa)
    ctx.call("hk_stream_destroy", sb)
