"""On-disk organ containers and the mixed catalog, over the library's C++
loader (hk_container.cpp), mirroring the reference's loaders:

  * organ_from_container(codec, payload) -- MixedPackedTensor::from_codec_payload
    (crates/hawking-core/src/model/qwen_complete_binary/q80_mixed_decode.rs:1336-1347)
  * organ_from_hq30(payload) -- HQ30UQ4 / HQ30G1B1 32-byte-header payloads
    (qwen_complete_binary/uniform_q4.rs:57-150, qwen_complete_binary/mod.rs:137-233)
  * MixedCatalog -- Qwen80MixedStreamingCatalog (model/qwen80_mixed_catalog.rs:176-555)
  * organ_from_q4_0(blocks, rows, cols) -- GGUF Q4_0 AoS blocks (dequant_q4_0, quant.rs:473-498)
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import (HK_BIN, HK_BIN_RICE, HK_Q4, HK_Q8, HK_U3, CatalogRecord)
from .organs import (BinaryGroupPacked, HgravS01LowRank, PackedOrgan, Qwen80Q4PackedTensor, RiceQ1Packed,
                     UniformFactor3, UniformFactorPacked)
from .runtime import Context

CODEC_BINARY, CODEC_RESIDUAL, CODEC_HGRAVS01, CODEC_UNIFORM8 = 0, 1, 2, 3
_BY_KIND = {HK_BIN: BinaryGroupPacked, HK_Q8: UniformFactorPacked, HK_BIN_RICE: RiceQ1Packed,
            HK_Q4: Qwen80Q4PackedTensor, HK_U3: UniformFactor3}


def _wrap(ctx: Context, h: C.c_void_p) -> PackedOrgan:
    kind = C.c_int32()
    ctx.check("hk_organ_info", ctx.L.hk_organ_info(h, C.byref(kind), None, None, None, None))
    return _BY_KIND[int(kind.value)]._wrap(ctx, h)


def _bound(ctx: Context, out: C.c_void_p, right: C.c_void_p):
    left = _wrap(ctx, out)
    if right.value:
        return HgravS01LowRank(left, _wrap(ctx, right))
    return left


def organ_from_container(ctx: Context, codec: int, payload: bytes):
    """A bound organ (or, for HGRAVS01, an HgravS01LowRank pair)."""
    buf = np.frombuffer(payload, np.uint8)
    out, right = C.c_void_p(), C.c_void_p()
    ctx.call("hk_organ_from_container", int(codec), buf.ctypes.data if buf.size else None, buf.size, ctx.stream,
             C.byref(out), C.byref(right))
    return _bound(ctx, out, right)


def organ_from_hq30(ctx: Context, payload: bytes) -> PackedOrgan:
    buf = np.frombuffer(payload, np.uint8)
    out = C.c_void_p()
    ctx.call("hk_organ_from_hq30", buf.ctypes.data, buf.size, ctx.stream, C.byref(out))
    return _wrap(ctx, out)


def organ_from_q4_0(ctx: Context, blocks, rows: int, cols: int) -> PackedOrgan:
    """GGUF Q4_0 blocks (18 bytes per 32 elements: f16 d, then 16 bytes of
    nibbles, element j low / j + 16 high) bound as a Q4 group-32 organ."""
    buf = np.ascontiguousarray(np.frombuffer(bytes(blocks), np.uint8) if not isinstance(blocks, np.ndarray)
                               else blocks.reshape(-1).view(np.uint8))
    out = C.c_void_p()
    ctx.call("hk_organ_from_q4_0", buf.ctypes.data, buf.size, rows, cols, ctx.stream, C.byref(out))
    return _wrap(ctx, out)


def _record(r: CatalogRecord) -> dict:
    return {"name": r.name.decode(), "codec": r.codec, "organ": r.organ, "shape": list(r.shape)[:r.ndim],
            "elements": r.elements, "segment_id": r.segment_id, "achieved_rank": r.achieved_rank,
            "offset": r.offset, "nbytes": r.nbytes, "sha256": bytes(r.sha256).hex(), "flags": r.flags,
            "n_fit_rows": r.n_fit_rows, "codec_bpw": r.codec_bpw}


class MixedCatalog:
    """An opened HQ80M15 catalog: records by name, payload windows of the
    mapped segments (SHA-256 checked on first use), and organs bound from them."""

    def __init__(self, ctx: Context, manifest_path: str):
        self.ctx = ctx
        h = C.c_void_p()
        ctx.call("hk_catalog_open", str(manifest_path).encode(), C.byref(h))
        self.h = h
        n, s, bpw, tpb = C.c_uint32(), C.c_uint32(), C.c_double(), C.c_uint64()
        ctx.check("hk_catalog_info", ctx.L.hk_catalog_info(h, C.byref(n), C.byref(s), C.byref(bpw), C.byref(tpb)))
        self.tensor_count, self.segment_count = int(n.value), int(s.value)
        self.complete_physical_bpw, self.tensor_payload_bytes = float(bpw.value), int(tpb.value)

    def records(self) -> list[dict]:
        out = []
        for i in range(self.tensor_count):
            r = CatalogRecord()
            self.ctx.check("hk_catalog_record_at", self.ctx.L.hk_catalog_record_at(self.h, i, C.byref(r)))
            out.append(_record(r))
        return out

    def record(self, name: str) -> dict:
        r = CatalogRecord()
        self.ctx.call("hk_catalog_find", self.h, name.encode(), C.byref(r))
        return _record(r)

    def payload(self, name: str, verify: bool = True) -> bytes:
        p, n = C.c_void_p(), C.c_size_t()
        self.ctx.call("hk_catalog_payload", self.h, name.encode(), int(verify), C.byref(p), C.byref(n))
        return C.string_at(p.value, n.value) if n.value else b""

    def load(self, name: str, verify: bool = True):
        """load_packed: the tensor bound as an organ (HGRAVS01: a low-rank pair)."""
        out, right = C.c_void_p(), C.c_void_p()
        self.ctx.call("hk_catalog_load", self.h, name.encode(), int(verify), self.ctx.stream, C.byref(out),
                      C.byref(right))
        return _bound(self.ctx, out, right)

    def close(self) -> None:
        if getattr(self, "h", None) and self.h.value:
            self.ctx.L.hk_catalog_close(self.h)
        self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
