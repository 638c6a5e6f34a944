"""hk_terminal_greedy_noalloc (no reference counterpart: the terminal head
for callers that cannot allocate) against hk_terminal_greedy, through the C
ABI: the same token and device status on two calls in a row, the second on
a smaller lm_head, for the fused q8 path and the unfused Q4 path."""
import ctypes as C
import sys

import numpy as np
import pytest

from tests import hk_testutil as U

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    from hawking_amd.runtime import Context
    return Context(0)


def _case(ctx, oracle, kind, vocab, hidden_n, n_valid, tag):
    from hawking_amd.head import TerminalHead
    from hawking_amd.organs import Qwen80Q4PackedTensor, UniformFactorPacked
    key = lambda k: oracle.stream_key(U.SEED, (0xA110C << 8) + 16 * tag + k)
    h = oracle.normal(key(1), hidden_n, 1.0)
    nw = oracle.normal(key(2), hidden_n, 0.02)
    w = oracle.normal(key(3), vocab * hidden_n, 0.05).reshape(vocab, hidden_n)
    if kind == "q8":
        s, c = oracle.uniform_pack(w, vocab, hidden_n, 8, 64)
        lm = UniformFactorPacked(ctx, s, c, vocab, hidden_n)
    else:
        s, c = oracle.q4_pack(w, 32)
        lm = Qwen80Q4PackedTensor(ctx, s, c, vocab, hidden_n, 32)
    return TerminalHead(ctx, nw, lm, n_valid), h


@pytest.mark.parametrize("kind", ["q8", "q4"])
def test_noalloc_head_matches_head(ctx, oracle, kind):
    shapes = [(151936, 1024, 151669), (4096, 512, 4000)]   # second call: a smaller lm_head
    for i, (vocab, hidden_n, n_valid) in enumerate(shapes):
        say("noalloc head", kind, vocab, hidden_n, n_valid)
        head, h = _case(ctx, oracle, kind, vocab, hidden_n, n_valid, i + (8 if kind == "q4" else 0))
        hd = ctx.to_device(h)
        ctx.device_status()
        head.greedy_device(hd)
        want = int(head.token.download()[0])
        want_status = ctx.device_status()
        tok = ctx.to_device(np.full(1, -7, np.int32))
        ctx.call("hk_terminal_greedy_noalloc", hd.ptr, head.norm_w.ptr, C.c_float(head.eps), head.lm_head.h,
                 n_valid, tok.ptr, ctx.stream)
        got = int(tok.download()[0])
        assert ctx.device_status() == want_status
        assert got == want, (kind, vocab, got, want)
        assert want == oracle.argmax_greedy(head.logits.download(), n_valid)


def test_noalloc_head_rejects_oversized_lm_head(ctx, oracle):
    from hawking_amd._lib import HK_E_UNSUPPORTED, HawkingError
    head, h = _case(ctx, oracle, "q8", 64, 9216, 64, 30)
    tok = ctx.empty(1, np.int32)
    with pytest.raises(HawkingError) as e:
        ctx.call("hk_terminal_greedy_noalloc", ctx.to_device(h).ptr, head.norm_w.ptr, C.c_float(1e-6),
                 head.lm_head.h, 64, tok.ptr, ctx.stream)
    assert e.value.code == HK_E_UNSUPPORTED
