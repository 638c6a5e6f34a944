"""The achievable-bandwidth control (hk_stream_control): every 16-byte word
of the buffer is read exactly once, whatever the slicing, and bad arguments
are rejected before a launch."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    from hawking_amd.runtime import Context
    return Context(0)


@pytest.mark.parametrize("n_floats,workgroups", [(1 << 20, 64), (1 << 20, 3), ((1 << 16) + 4, 7), (4, 5)])
def test_stream_control_reads_every_word_once(ctx, n_floats, workgroups):
    say("stream control", n_floats, workgroups)
    data = ctx.to_device(np.ones(n_floats, np.float32))
    out = ctx.empty(workgroups)
    ctx.call("hk_stream_control", data.ptr, n_floats * 4, out.ptr, workgroups, ctx.stream)
    sums = out.download()
    # each slice's sum counts its floats (exact: < 2^24); together every float once
    assert float(sums.astype(np.float64).sum()) == float(n_floats)
    assert np.all(sums >= 0) and np.all(sums == np.round(sums))


def test_stream_control_rejects_bad_arguments(ctx):
    from hawking_amd._lib import HK_E_INVALID_ARG, HawkingError
    data = ctx.empty(64)
    out = ctx.empty(4)
    for nbytes, wg in ((0, 4), (20, 4), (256, 0)):
        with pytest.raises(HawkingError) as e:
            ctx.call("hk_stream_control", data.ptr, nbytes, out.ptr, wg, ctx.stream)
        assert e.value.code == HK_E_INVALID_ARG
