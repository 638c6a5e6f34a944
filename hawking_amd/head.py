"""The device-side terminal head: final RMSNorm(1+w) -> lm_head -> greedy
token, mirroring terminal_greedy
(crates/hawking-core/src/model/qwen80_mixed_hybrid_decode.rs:3754-3790) over
hk_terminal_greedy.  The token id is produced on the device; `greedy` copies
it back only for host callers."""
from __future__ import annotations

import numpy as np

from .organs import PackedOrgan
from .runtime import Context, DeviceArray

QWEN80_VOCAB = 151_936            # lm_head rows (qwen80_complete_runtime.rs:62)
QWEN80_TOKENIZER_VOCAB = 151_669  # rows a token can come from (qwen80_complete_runtime.rs:66)
QWEN80_RMS_EPS = 1.0e-6


class TerminalHead:
    """model.norm.weight + lm_head.weight bound on the device, with the
    workspaces (normalised hidden state, logits, pick key, token) the call
    writes.  Heads that share an lm_head but not these workspaces may run on
    different streams at once."""

    def __init__(self, ctx: Context, norm_w: np.ndarray, lm_head: PackedOrgan,
                 n_valid: int | None = None, eps: float = QWEN80_RMS_EPS):
        norm_w = np.ascontiguousarray(norm_w, np.float32)
        if norm_w.shape != (lm_head.cols,):
            raise ValueError("norm weight length must equal lm_head cols")
        self.ctx, self.lm_head, self.eps = ctx, lm_head, float(eps)
        self.n_valid = lm_head.rows if n_valid is None else int(n_valid)
        self.norm_w = ctx.to_device(norm_w)
        self.xn = ctx.empty(lm_head.cols)
        self.logits = ctx.empty(lm_head.rows)
        self.token = ctx.empty(1, np.int32)
        # the pick's 16-byte key slot: zero before the first call, left zeroed by each call
        self.pick = ctx.to_device(np.zeros(2, np.uint64))

    def greedy_device(self, hidden, token=None, stream=None) -> None:
        """Enqueue the head; the token lands in `token` (or self.token)."""
        out = self.token if token is None else token
        hp = hidden.ptr if isinstance(hidden, DeviceArray) else hidden
        tp = out.ptr if isinstance(out, DeviceArray) else out
        self.ctx.call("hk_terminal_greedy", hp, self.norm_w.ptr, self.eps, self.lm_head.h, self.n_valid,
                      self.xn.ptr, self.logits.ptr, self.pick.ptr, tp,
                      stream if stream is not None else self.ctx.stream)

    def greedy(self, hidden: np.ndarray) -> int:
        """Host convenience: upload, run, synchronise; HawkingError
        (HK_E_NONFINITE) when the device flagged a non-finite value."""
        from ._lib import HK_E_NONFINITE, HawkingError
        self.ctx.device_status()  # start from a clear status
        self.greedy_device(self.ctx.to_device(np.ascontiguousarray(hidden, np.float32)))
        if self.ctx.device_status() & 1:
            raise HawkingError("hk_terminal_greedy", HK_E_NONFINITE, "a non-finite value or no finite logit")
        return int(self.token.download()[0])
