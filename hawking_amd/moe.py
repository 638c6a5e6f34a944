"""Routers and the MoE decode step on the GPU.

Mirrors the reference's routing and MoE-suffix API:
  * source_qwen80_topk_router (crates/hawking-core/src/model/qwen80_complete_runtime.rs:5970-6025)
  * topk_softmax_batch        (crates/hawking-core/src/kernels/mod.rs:342-374)
  * noaux_tc router           (crates/hawking-core/src/gravity_glm.rs:447-500)
  * moe_suffix                (crates/hawking-core/src/model/qwen80_uniform_q4_hybrid_decode.rs:2615-2757)
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import HK_MIXED, HK_Q4, MoeConfig, MoeLayerSrc, OrganSrc
from .runtime import Context, DeviceArray


def _pp(a):
    """Device pointer of a DeviceArray, a raw c_void_p, or None."""
    if a is None:
        return None
    return a.ptr if isinstance(a, DeviceArray) else a


def _dev(ctx: Context, a) -> DeviceArray:
    return a if isinstance(a, DeviceArray) else ctx.to_device(np.ascontiguousarray(a, np.float32))


def topk_router(ctx: Context, logits, top_k: int, tie_eps: float = 0.0, renorm: bool = True,
                n_tokens: int = 1):
    """Softmax top-k on device; returns (ids, weights) as numpy (synchronises)."""
    ld = _dev(ctx, logits)
    n_experts = ld.shape[-1] if n_tokens == 1 else ld.shape[-1]
    ids = ctx.empty(n_tokens * top_k, np.int32)
    w = ctx.empty(n_tokens * top_k, np.float32)
    ctx.call("hk_router_softmax_topk", ld.ptr, n_tokens, n_experts, top_k, tie_eps, int(renorm),
             ids.ptr, w.ptr, ctx.stream)
    return ids.download().reshape(n_tokens, top_k), w.download().reshape(n_tokens, top_k)


def source_qwen80_topk_router(ctx: Context, logits, top_k: int = 10):
    ids, w = topk_router(ctx, logits, top_k, 0.0, True)
    return ids[0], w[0]


def noaux_tc_router(ctx: Context, logits, bias, n_group: int, topk_group: int, top_k: int,
                    norm_topk_prob: bool = True, routed_scaling_factor: float = 1.0, n_tokens: int = 1):
    ld = _dev(ctx, logits)
    bd = _dev(ctx, bias)
    n_experts = int(np.prod(ld.shape)) // n_tokens
    ids = ctx.empty(n_tokens * top_k, np.int32)
    w = ctx.empty(n_tokens * top_k, np.float32)
    ctx.call("hk_router_noaux_tc", ld.ptr, bd.ptr, n_tokens, n_experts, n_group, topk_group, top_k,
             int(norm_topk_prob), routed_scaling_factor, ids.ptr, w.ptr, ctx.stream)
    return ids.download().reshape(n_tokens, top_k), w.download().reshape(n_tokens, top_k)


# stream-id projections (hk_moe_stream_id)
PROJ_GATE, PROJ_UP, PROJ_DOWN = 0, 1, 2
PROJ_NORM, PROJ_ROUTER, PROJ_SHARED_GATE, PROJ_COIN = 16, 17, 18, 32


def moe_stream_id(layer: int, expert: int, proj: int) -> int:
    return ((layer + 1) << 40) | (expert << 8) | proj


@dataclass
class MoeShape:
    n_layers: int = 1
    hidden: int = 2048
    inter: int = 512
    shared_inter: int = 512
    n_experts: int = 512
    top_k: int = 10
    expert_kind: int = HK_Q4
    expert_group: int = 32
    shared_gate: bool = True
    eps: float = 1e-6
    router: int = 0             # HK_ROUTER_SOFTMAX (decode path) or HK_ROUTER_NOAUX_TC (batched block)
    n_group: int = 1            # noaux_tc
    topk_group: int = 1
    norm_topk_prob: bool = True
    routed_scaling_factor: float = 1.0
    route_tie_eps: float = 0.0  # softmax router tie window (route_tie_epsilon, moe.rs:8-14); 0 = strict
    stack_launch: int = 0       # HK_STACK_PER_LAYER (0) or HK_STACK_PERSISTENT (1)

    @classmethod
    def deepseek_v3(cls, n_layers=1, n_group=1, topk_group=1, **kw):
        """The DeepSeek-V3-shaped batched block: hidden 7168, 256 experts x 2048
        (Q4 G32) + 1 shared, top-8 noaux_tc (norm, x2.5)."""
        base = dict(n_layers=n_layers, hidden=7168, inter=2048, shared_inter=2048, n_experts=256, top_k=8,
                    expert_kind=HK_Q4, expert_group=32, shared_gate=False, router=1, n_group=n_group,
                    topk_group=topk_group, norm_topk_prob=True, routed_scaling_factor=2.5)
        base.update(kw)
        return cls(**base)


class MoeModel:
    """Device-resident MoE stack: per layer RMSNorm(1+w) weight, f32 router,
    optional shared-expert gate, and the packed expert table."""

    def __init__(self, ctx: Context, shape: MoeShape):
        self.ctx, self.shape = ctx, shape
        cfg = MoeConfig(shape.n_layers, shape.hidden, shape.inter, shape.shared_inter, shape.n_experts,
                        shape.top_k, shape.expert_kind, shape.expert_group, int(shape.shared_gate), shape.eps,
                        shape.router, shape.n_group, shape.topk_group, int(shape.norm_topk_prob),
                        shape.routed_scaling_factor, shape.route_tie_eps, shape.stack_launch)
        h = C.c_void_p()
        ctx.call("hk_moe_model_create", C.byref(cfg), C.byref(h))
        self.h = h

    def free(self):
        if getattr(self, "h", None) and self.h.value and self.ctx.h:
            self.ctx.L.hk_moe_model_free(self.ctx.h, self.h)
        self.h = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def fill_synthetic(self, seed: int) -> None:
        self.ctx.call("hk_moe_model_fill_synthetic", self.h, seed, self.ctx.stream)

    def set_layer(self, layer: int, norm_w, router_w, experts, shared=None, shared_gate_w=None,
                  router_bias=None) -> None:
        """experts: list over expert id of (gate, up, down) canonical organ dicts
        (see organ_src); shared likewise or None."""
        keep = []

        def arr(a, dt):
            a = np.ascontiguousarray(a, dt)
            keep.append(a)
            return a.ctypes.data

        def src(d) -> OrganSrc:
            if d["kind"] == HK_Q4:
                return OrganSrc(kind=HK_Q4, group=d["group"], rows=d["rows"], cols=d["cols"],
                                scales=arr(d["scales"], np.uint16), codes=arr(d["codes"], np.uint8))
            return OrganSrc(kind=HK_MIXED, group=128, rows=d["rows"], cols=d["cols"],
                            tags=arr(d["tags"], np.uint8),
                            scales=arr(d["bin_scales"], np.uint16) if d["bin_scales"].size else None,
                            codes=arr(d["bin_signs"], np.uint8) if d["bin_signs"].size else None,
                            q2_scales=arr(d["q2_scales"], np.uint16) if d["q2_scales"].size else None,
                            q2_codes=arr(d["q2_codes"], np.uint8) if d["q2_codes"].size else None,
                            n_bin=d["bin_scales"].size, n_q2=d["q2_scales"].size // 2)

        ex = (OrganSrc * (len(experts) * 3))()
        for e, trip in enumerate(experts):
            for j in range(3):
                ex[e * 3 + j] = src(trip[j])
        sh = None
        if shared is not None:
            sh = (OrganSrc * 3)(*[src(d) for d in shared])
        L = MoeLayerSrc(arr(norm_w, np.float32), arr(router_w, np.float32),
                        arr(shared_gate_w, np.float32) if shared_gate_w is not None else None,
                        C.cast(ex, C.c_void_p), C.cast(sh, C.c_void_p) if sh is not None else None,
                        arr(router_bias, np.float32) if router_bias is not None else None)
        self.ctx.call("hk_moe_model_set_layer", self.h, layer, C.byref(L), self.ctx.stream)

    def expert_bytes(self, layer: int, expert: int) -> int:
        b = C.c_size_t()
        self.ctx.check("hk_moe_expert_bytes", self.ctx.L.hk_moe_expert_bytes(self.h, layer, expert, C.byref(b)))
        return int(b.value)

    def model_bytes(self) -> tuple[int, int]:
        a, b = C.c_size_t(), C.c_size_t()
        self.ctx.check("hk_moe_model_bytes", self.ctx.L.hk_moe_model_bytes(self.h, C.byref(a), C.byref(b)))
        return int(a.value), int(b.value)

    # -- decode -----------------------------------------------------------------------
    def decode_layer_device(self, layer: int, h_in: DeviceArray, h_out: DeviceArray,
                            ids: DeviceArray | None = None, weights: DeviceArray | None = None,
                            stream=None) -> None:
        self.ctx.call("hk_moe_decode_layer", self.h, layer, _pp(h_in), _pp(h_out),
                      _pp(ids), _pp(weights),
                      stream if stream is not None else self.ctx.stream)

    def decode_stack_device(self, h_in: DeviceArray, h_out: DeviceArray, ids: DeviceArray | None = None,
                            weights: DeviceArray | None = None, stream=None) -> None:
        self.ctx.call("hk_moe_decode_stack", self.h, _pp(h_in), _pp(h_out),
                      _pp(ids), _pp(weights),
                      stream if stream is not None else self.ctx.stream)

    def set_stack_launch(self, mode: int) -> None:
        """HK_STACK_PER_LAYER (0) or HK_STACK_PERSISTENT (1) for decode_stack (hk_moe_model_set_stack_launch)."""
        self.ctx.call("hk_moe_model_set_stack_launch", self.h, int(mode))
        self.shape.stack_launch = int(mode)

    def set_stall_polls(self, polls: int) -> None:
        """The persistent launch's bound on each hand-off wait (hk_moe_model_set_stall_polls)."""
        self.ctx.call("hk_moe_model_set_stall_polls", self.h, int(polls))

    def stack_is_persistent(self) -> bool:
        """Whether decode_stack runs as one persistent launch here (hk_moe_decode_stack_persistent)."""
        v = C.c_int(0)
        self.ctx.call("hk_moe_decode_stack_persistent", self.h, C.byref(v))
        return bool(v.value)

    def moe_block_device(self, layer: int, route_ids: DeviceArray, route_weights: DeviceArray, n_routes: int,
                         x: DeviceArray, out: DeviceArray, include_shared: bool = True, stream=None) -> None:
        """BackendMoe::moe_block: out += sum_r w_r mlp_r(x) (+ g mlp_shared(x)),
        routes supplied by the caller on the device (hk_moe_block)."""
        self.ctx.call("hk_moe_block", self.h, layer, _pp(route_ids), _pp(route_weights), n_routes,
                      int(include_shared), _pp(x), _pp(out), stream if stream is not None else self.ctx.stream)

    def moe_block(self, layer: int, route_ids, route_weights, x: np.ndarray, out: np.ndarray | None = None,
                  include_shared: bool = True) -> np.ndarray:
        """Host convenience of moe_block_device: returns out + combined (out
        defaults to zeros)."""
        ids = self.ctx.to_device(np.ascontiguousarray(route_ids, np.int32))
        w = self.ctx.to_device(np.ascontiguousarray(route_weights, np.float32))
        xd = self.ctx.to_device(np.ascontiguousarray(x, np.float32))
        o = np.zeros(self.shape.hidden, np.float32) if out is None else np.ascontiguousarray(out, np.float32)
        od = self.ctx.to_device(o)
        self.moe_block_device(layer, ids, w, int(ids.shape[0]), xd, od, include_shared)
        return od.download()

    def moe_suffix(self, layer: int, h: np.ndarray):
        """One layer on numpy input: returns (out, ids, weights)."""
        hd = self.ctx.to_device(np.ascontiguousarray(h, np.float32))
        out = self.ctx.empty(self.shape.hidden)
        ids = self.ctx.empty(self.shape.top_k, np.int32)
        w = self.ctx.empty(self.shape.top_k, np.float32)
        self.decode_layer_device(layer, hd, out, ids, w)
        return out.download(), ids.download(), w.download()

    def forward_token(self, h: np.ndarray):
        """All layers: returns (out, ids[n_layers, k], weights[n_layers, k])."""
        s = self.shape
        hd = self.ctx.to_device(np.ascontiguousarray(h, np.float32))
        out = self.ctx.empty(s.hidden)
        ids = self.ctx.empty(s.n_layers * s.top_k, np.int32)
        w = self.ctx.empty(s.n_layers * s.top_k, np.float32)
        self.decode_stack_device(hd, out, ids, w)
        return (out.download(), ids.download().reshape(s.n_layers, s.top_k),
                w.download().reshape(s.n_layers, s.top_k))

    # -- batched noaux_tc block ------------------------------------------------------
    def forward_batch_device(self, layer: int, x_bf16: DeviceArray, n_tokens: int, y: DeviceArray,
                             ids: DeviceArray | None = None, weights: DeviceArray | None = None, stream=None) -> None:
        self.ctx.call("hk_moe_forward_batch", self.h, layer, _pp(x_bf16), n_tokens, _pp(y), _pp(ids), _pp(weights),
                      stream if stream is not None else self.ctx.stream)

    def routed_moe(self, layer: int, x_bf16: np.ndarray):
        """routed_moe for a batch: x_bf16 uint16 [T, hidden] (bf16 bits).
        Returns (y [T, hidden] f32, ids [T, top_k], weights [T, top_k])."""
        s = self.shape
        x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
        T = x_bf16.shape[0]
        xd = self.ctx.to_device(x_bf16)
        y = self.ctx.empty((T, s.hidden))
        ids = self.ctx.empty((T, s.top_k), np.int32)
        w = self.ctx.empty((T, s.top_k), np.float32)
        self.forward_batch_device(layer, xd, T, y, ids, w)
        return y.download(), ids.download(), w.download()


class Mixed15Layer:
    """One MoE layer of the mixed-1p5-v1 artifact over bound organs
    (moe_suffix, model/qwen80_mixed_hybrid_decode.rs:3636-3752, with
    routed_wave :2192-2386).

    experts: per expert (gate BinaryGroupPacked, up RiceQ1Packed, down) with
    down an HgravS01LowRank or its (left, right) factor organs; router /
    shared_gate / shared (gate, up, down):
    PackedOrgan (HGRAVU01 q8 in the artifact).  The layer keeps references
    to the organs; they must outlive it."""

    def __init__(self, ctx: Context, norm_w, router, experts, top_k: int, shared=None, shared_gate=None,
                 eps: float = 1e-6, route_tie_eps: float = 0.0):
        from ._lib import Moe15LayerSrc
        self.ctx = ctx
        self.h = None
        downs = [t[2] if isinstance(t[2], tuple) else (t[2].left, t[2].right) for t in experts]
        g0 = experts[0][0]
        self.hidden, self.inter, self.n_experts, self.top_k = downs[0][0].rows, g0.rows, len(experts), top_k
        self.rank = downs[0][0].cols
        self.shared_inter = shared[0].rows if shared is not None else 0
        self._keep = (router, experts, shared, shared_gate)
        self._norm = np.ascontiguousarray(norm_w, np.float32)
        E = self.n_experts
        tab = [(C.c_void_p * E)(*[t[0].h.value for t in experts]),
               (C.c_void_p * E)(*[t[1].h.value for t in experts]),
               (C.c_void_p * E)(*[d[0].h.value for d in downs]),
               (C.c_void_p * E)(*[d[1].h.value for d in downs])]
        self._tab = tab
        sh = shared if shared is not None else (None, None, None)
        src = Moe15LayerSrc(hidden=self.hidden, inter=self.inter, shared_inter=self.shared_inter, n_experts=E,
                            top_k=top_k, eps=eps, route_tie_eps=route_tie_eps, norm_w=self._norm.ctypes.data,
                            router=router.h,
                            shared_gate=shared_gate.h if shared_gate is not None else None,
                            shared_gate_proj=sh[0].h if sh[0] is not None else None,
                            shared_up=sh[1].h if sh[1] is not None else None,
                            shared_down=sh[2].h if sh[2] is not None else None,
                            gate=C.cast(tab[0], C.c_void_p), up=C.cast(tab[1], C.c_void_p),
                            down_left=C.cast(tab[2], C.c_void_p), down_right=C.cast(tab[3], C.c_void_p))
        h = C.c_void_p()
        ctx.call("hk_moe15_layer_create", C.byref(src), C.byref(h))
        self.h = h

    def free(self):
        if self.h is not None:
            self.ctx.call("hk_moe15_layer_free", self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def decode_device(self, h_in, h_out, ids=None, weights=None, stream=None) -> None:
        self.ctx.call("hk_moe15_decode_layer", self.h, _pp(h_in), _pp(h_out), _pp(ids), _pp(weights),
                      stream if stream is not None else self.ctx.stream)

    def moe_suffix(self, h: np.ndarray):
        """One layer on numpy input: returns (out, ids, weights)."""
        hd = self.ctx.to_device(np.ascontiguousarray(h, np.float32))
        out = self.ctx.empty(self.hidden)
        ids = self.ctx.empty(self.top_k, np.int32)
        w = self.ctx.empty(self.top_k, np.float32)
        self.decode_device(hd, out, ids, w)
        return out.download(), ids.download(), w.download()


def mixed15_decode_stack(ctx: Context, layers: list[Mixed15Layer], h_in, h_out, ids=None, weights=None,
                         stream=None) -> None:
    """All layers for one token on device data (hk_moe15_decode_stack)."""
    arr = (C.c_void_p * len(layers))(*[l.h.value for l in layers])
    ctx.call("hk_moe15_decode_stack", arr, len(layers), _pp(h_in), _pp(h_out), _pp(ids), _pp(weights),
             stream if stream is not None else ctx.stream)


# ---------------------------------------------------------------- synthetic mixed-1p5-v1 model
# The reference's measured artifact is a Qwen3-Next-80B-A3B pack whose experts
# mix three codecs per tensor (q80_mixed_decode.rs:7-21,
# qwen80_mixed_catalog.rs:30-33): gate HGRAVB01, up HGRAVR02 (2 % Rice
# residual), down HGRAVS01 (rank-160 3-bit factors); router, shared-expert
# gate and shared expert HGRAVU01 q8.  The synthetic stand-in draws every
# tensor from the counter-based generator on the device (no checkpoint is
# available), so the oracle can regenerate any one of them.
MIXED15_GATE, MIXED15_UP, MIXED15_DOWN_LEFT, MIXED15_DOWN_RIGHT = 0, 1, 2, 3
MIXED15_ROUTER, MIXED15_SHARED_GATE, MIXED15_SHARED_GATE_PROJ, MIXED15_SHARED_UP, MIXED15_SHARED_DOWN = 16, 17, 18, 19, 20
MIXED15_NORM = 21


@dataclass
class Mixed15Dims:
    hidden: int = 2048
    inter: int = 512
    shared_inter: int = 512
    n_experts: int = 512
    top_k: int = 10
    rank: int = 160
    eps: float = 1e-6


def mixed15_stream_id(layer: int, expert: int, proj: int) -> int:
    """Generator stream of one tensor of the synthetic mixed-1p5 model; expert
    n_experts holds the router, the shared gate and the shared expert."""
    return (0xC15 << 40) | (layer << 24) | (expert << 8) | proj


def mixed15_tensor(d: Mixed15Dims, expert: int, proj: int):
    """(kind, rows, cols, group, sigma) of one synthetic tensor."""
    from ._lib import HK_BIN, HK_BIN_RICE, HK_Q8, HK_U3
    H, I, SI, E, r = d.hidden, d.inter, d.shared_inter, d.n_experts, d.rank
    table = {
        MIXED15_GATE: (HK_BIN, I, H, 128, 0.02),
        MIXED15_UP: (HK_BIN_RICE, I, H, 128, 0.02),
        MIXED15_DOWN_LEFT: (HK_U3, H, r, 64, 0.05),
        MIXED15_DOWN_RIGHT: (HK_U3, r, I, 64, 0.02),
        MIXED15_ROUTER: (HK_Q8, E, H, 64, 0.02),
        MIXED15_SHARED_GATE: (HK_Q8, 1, H, 64, 0.02),
        MIXED15_SHARED_GATE_PROJ: (HK_Q8, SI, H, 64, 0.02),
        MIXED15_SHARED_UP: (HK_Q8, SI, H, 64, 0.02),
        MIXED15_SHARED_DOWN: (HK_Q8, H, SI, 64, 0.02),
    }
    return table[proj]


def synthetic_mixed15_layers(ctx: Context, seed: int, n_layers: int, d: Mixed15Dims = Mixed15Dims(),
                             route_tie_eps: float = 0.0):
    """n_layers synthetic mixed-1p5 layers generated and packed on the device.
    Returns (layers, expert_bytes[l][e] = packed bytes of expert e's four
    organs, dense_bytes[l] = router + shared gate + shared expert + norm)."""
    from .organs import SyntheticOrgan, stream_key
    layers, expert_bytes, dense_bytes = [], [], []
    E = d.n_experts
    nbuf = ctx.empty(d.hidden)
    for l in range(n_layers):
        def syn(e, p):
            kind, rows, cols, group, sigma = mixed15_tensor(d, e, p)
            return SyntheticOrgan(ctx, kind, rows, cols, stream_key(seed, mixed15_stream_id(l, e, p)), 0,
                                  group=group, sigma=sigma)
        experts = [(syn(e, MIXED15_GATE), syn(e, MIXED15_UP), (syn(e, MIXED15_DOWN_LEFT), syn(e, MIXED15_DOWN_RIGHT)))
                   for e in range(E)]
        router = syn(E, MIXED15_ROUTER)
        sgate = shared = None
        if d.shared_inter:
            sgate = syn(E, MIXED15_SHARED_GATE)
            shared = (syn(E, MIXED15_SHARED_GATE_PROJ), syn(E, MIXED15_SHARED_UP), syn(E, MIXED15_SHARED_DOWN))
        ctx.call("hk_synth_normal", stream_key(seed, mixed15_stream_id(l, E, MIXED15_NORM)), 0, d.hidden, 0.02,
                 nbuf.ptr, ctx.stream)
        nw = nbuf.download()
        layers.append(Mixed15Layer(ctx, nw, router, experts, d.top_k, shared=shared, shared_gate=sgate, eps=d.eps,
                                   route_tie_eps=route_tie_eps))
        expert_bytes.append([t[0].packed_bytes + t[1].packed_bytes + t[2][0].packed_bytes + t[2][1].packed_bytes
                             for t in experts])
        dense_bytes.append(router.packed_bytes + d.hidden * 4 +
                           ((sgate.packed_bytes + sum(o.packed_bytes for o in shared)) if shared else 0))
    return layers, expert_bytes, dense_bytes


def mixed15_forward_token(ctx: Context, layers: list[Mixed15Layer], h: np.ndarray):
    """All layers for one token on numpy input through hk_moe15_decode_stack:
    returns (out, ids[n_layers, k], weights[n_layers, k])."""
    H, K, n = layers[0].hidden, layers[0].top_k, len(layers)
    hd = ctx.to_device(np.ascontiguousarray(h, np.float32))
    out = ctx.empty(H)
    ids = ctx.empty(n * K, np.int32)
    w = ctx.empty(n * K, np.float32)
    mixed15_decode_stack(ctx, layers, hd, out, ids, w)
    return out.download(), ids.download().reshape(n, K), w.download().reshape(n, K)
