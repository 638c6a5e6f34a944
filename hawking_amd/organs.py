"""Packed matvec organs on the GPU, mirroring hawking-core's organ API.

Reference names are kept where the reference has them:
  * Qwen80Q4PackedTensor.matvec / gather_row
    (crates/hawking-core/src/model/qwen80_uniform_q4_hybrid_decode.rs:900-1036)
  * BinaryGroupPacked + binary_group_matvec_f32
    (crates/hawking-core/src/model/qwen_complete_binary/q80_mixed_decode.rs:48-257)
  * MixedPackedTensor (q80_mixed_decode.rs:1073-1417)
  * UniformFactorPacked + uniform_factor_matvec_f32 at 8 bits, group 64
    (HGRAVU01, q80_mixed_decode.rs:529-612,1047-1070)
  * HGRAVS01 low-rank: two 3-bit uniform factors and
    hgravs01_two_stage_matvec_f32 (q80_mixed_decode.rs:614-629,1019-1046)
  * RiceQ1Packed + binary_rice_q1_matvec_f32 (HGRAVR02: binary base plus a
    Rice-coded 1-bit residual, q80_mixed_decode.rs:60-69,383-527)
Every matvec runs the gfx950 kernels through the C ABI; the inputs are the
reference's canonical packed bytes, uploaded and repacked once.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import HK_BIN, HK_BIN_RICE, HK_F32, HK_MIXED, HK_Q4, HK_Q8, HK_U3, OrganSrc, RiceQ1Src
from .runtime import Context, DeviceArray


def _ptr(a):
    return None if a is None else np.ascontiguousarray(a).ctypes.data


class PackedOrgan:
    """One packed matrix resident in device memory (library-owned)."""

    kind: int = -1

    def __init__(self, ctx: Context, src: OrganSrc, keep: tuple):
        self.ctx = ctx
        h = C.c_void_p()
        ctx.call("hk_organ_upload", C.byref(src), ctx.stream, C.byref(h))
        self.h = h
        self.rows, self.cols, self.group = int(src.rows), int(src.cols), int(src.group)
        del keep  # host buffers only had to outlive the synchronous upload
        sz = C.c_size_t()
        ctx.check("hk_organ_info", ctx.L.hk_organ_info(h, None, None, None, None, C.byref(sz)))
        self.packed_bytes = int(sz.value)

    @classmethod
    def _wrap(cls, ctx: Context, h: C.c_void_p) -> "PackedOrgan":
        """An object of this class around an organ the library already built
        (the loaders); shape and bytes come from hk_organ_info."""
        self = cls.__new__(cls)
        self.ctx, self.h = ctx, h
        kind, group, rows, cols, sz = C.c_int32(), C.c_int32(), C.c_uint32(), C.c_uint32(), C.c_size_t()
        ctx.check("hk_organ_info", ctx.L.hk_organ_info(h, C.byref(kind), C.byref(group), C.byref(rows),
                                                         C.byref(cols), C.byref(sz)))
        self.kind, self.group = int(kind.value), int(group.value)
        self.rows, self.cols, self.packed_bytes = int(rows.value), int(cols.value), int(sz.value)
        return self

    def free(self):
        if getattr(self, "h", None) and self.h.value and self.ctx.h:
            self.ctx.L.hk_organ_free(self.ctx.h, self.h)
        self.h = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    # -- device-pointer API --------------------------------------------------------
    def matvec_device(self, x: DeviceArray | C.c_void_p, y: DeviceArray | C.c_void_p, stream=None) -> None:
        xp = x.ptr if isinstance(x, DeviceArray) else x
        yp = y.ptr if isinstance(y, DeviceArray) else y
        self.ctx.call("hk_gemv", self.h, xp, yp, stream if stream is not None else self.ctx.stream)

    def decode_rows_device(self, row0: int, nrows: int, out: DeviceArray, stream=None) -> None:
        self.ctx.call("hk_decode_rows", self.h, row0, nrows, out.ptr,
                      stream if stream is not None else self.ctx.stream)

    # -- numpy convenience (uploads, runs, synchronises) -----------------------------
    def matvec(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        if x.shape != (self.cols,):
            raise ValueError(f"matvec input {x.shape} != cols {self.cols}")
        xd = self.ctx.to_device(x)
        yd = self.ctx.empty(self.rows)
        self.matvec_device(xd, yd)
        return yd.download()

    def decode(self, row0: int = 0, nrows: int | None = None) -> np.ndarray:
        nrows = self.rows - row0 if nrows is None else nrows
        out = self.ctx.empty((nrows, self.cols))
        self.decode_rows_device(row0, nrows, out)
        return out.download()

    def gather_row(self, row: int) -> np.ndarray:
        return self.decode(row, 1)[0]


class Qwen80Q4PackedTensor(PackedOrgan):
    """Uniform Q4 (HQ30UQ4 semantics), group 32/64/128."""

    kind = HK_Q4

    def __init__(self, ctx: Context, scales: np.ndarray, codes: np.ndarray, rows: int, cols: int,
                 group: int):
        scales = np.ascontiguousarray(scales, np.uint16)
        codes = np.ascontiguousarray(codes, np.uint8)
        if scales.size != rows * cols // max(group, 1) or codes.size != rows * cols // 2:
            raise ValueError("Q4 scales/codes sizes disagree with the shape")
        src = OrganSrc(kind=HK_Q4, group=group, rows=rows, cols=cols, scales=_ptr(scales), codes=_ptr(codes))
        super().__init__(ctx, src, (scales, codes))


class BinaryGroupPacked(PackedOrgan):
    """Binary sign plane, group 128 (HGRAVB01 body)."""

    kind = HK_BIN

    def __init__(self, ctx: Context, scales: np.ndarray, signs: np.ndarray, rows: int, cols: int):
        scales = np.ascontiguousarray(scales, np.uint16)
        signs = np.ascontiguousarray(signs, np.uint8)
        if scales.size != rows * cols // 128 or signs.size != rows * cols // 8:
            raise ValueError("binary scales/signs sizes disagree with the shape")
        src = OrganSrc(kind=HK_BIN, group=128, rows=rows, cols=cols, scales=_ptr(scales), codes=_ptr(signs))
        super().__init__(ctx, src, (scales, signs))


def binary_group_matvec_f32(packed: BinaryGroupPacked, x: np.ndarray) -> np.ndarray:
    """GPU counterpart of binary_group_matvec_f32 (q80_mixed_decode.rs:245-257)."""
    return packed.matvec(x)


class UniformFactorPacked(PackedOrgan):
    """Uniform 8-bit, group 64 (HGRAVU01 body): scales f16[rows*cols/64] and
    codes u8[rows*cols] (code = q + 127)."""

    kind = HK_Q8

    def __init__(self, ctx: Context, scales: np.ndarray, codes: np.ndarray, rows: int, cols: int):
        scales = np.ascontiguousarray(scales, np.uint16)
        codes = np.ascontiguousarray(codes, np.uint8)
        if scales.size != rows * cols // 64 or codes.size != rows * cols:
            raise ValueError("q8 scales/codes sizes disagree with the shape")
        src = OrganSrc(kind=HK_Q8, group=64, rows=rows, cols=cols, scales=_ptr(scales), codes=_ptr(codes))
        super().__init__(ctx, src, (scales, codes))


def uniform_factor_matvec_f32(packed: UniformFactorPacked, x: np.ndarray) -> np.ndarray:
    """GPU counterpart of uniform_factor_matvec_f32 (q80_mixed_decode.rs:600-612)."""
    return packed.matvec(x)


class UniformFactor3(PackedOrgan):
    """Uniform 3-bit factor, flat groups of 64 (an HGRAVS01 factor body):
    scales f16[ceil(rows*cols/64)] and 24 code bytes per group (LSB-first,
    code = q + 3).  Needs cols % 32 == 0."""

    kind = HK_U3

    def __init__(self, ctx: Context, scales: np.ndarray, codes: np.ndarray, rows: int, cols: int):
        scales = np.ascontiguousarray(scales, np.uint16)
        codes = np.ascontiguousarray(codes, np.uint8)
        groups = (rows * cols + 63) // 64
        if scales.size != groups or codes.size != groups * 24:
            raise ValueError("3-bit factor scales/codes sizes disagree with the shape")
        src = OrganSrc(kind=HK_U3, group=64, rows=rows, cols=cols, scales=_ptr(scales), codes=_ptr(codes))
        super().__init__(ctx, src, (scales, codes))


class HgravS01LowRank:
    """W ~= L R with L rows x rank and R rank x cols (HGRAVS01): y = L (R x)
    as two launches through a device mid vector of `rank` floats."""

    def __init__(self, left: UniformFactor3, right: UniformFactor3):
        if right.rows != left.cols:
            raise ValueError("right rows (the rank) must equal left cols")
        self.left, self.right = left, right
        self.ctx = left.ctx
        self.rows, self.rank, self.cols = left.rows, left.cols, right.cols
        self.mid = self.ctx.empty(self.rank)

    def matvec_device(self, x: DeviceArray, y: DeviceArray, stream=None) -> None:
        self.ctx.call("hk_gemv_lowrank", self.left.h, self.right.h, x.ptr, self.mid.ptr, y.ptr,
                      stream if stream is not None else self.ctx.stream)

    def matvec(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        if x.shape != (self.cols,):
            raise ValueError(f"matvec input {x.shape} != cols {self.cols}")
        xd = self.ctx.to_device(x)
        yd = self.ctx.empty(self.rows)
        self.matvec_device(xd, yd)
        return yd.download()


def hgravs01_two_stage_matvec_f32(packed: HgravS01LowRank, x: np.ndarray) -> np.ndarray:
    """GPU counterpart of hgravs01_two_stage_matvec_f32 (q80_mixed_decode.rs:614-629)."""
    return packed.matvec(x)


class RiceQ1Packed(PackedOrgan):
    """HGRAVR02 organ from its canonical body: binary group-128 base
    (bin_scales, bin_signs), first_index + Rice(gaps) with rice_k, one sign
    bit per outlier and the f16 residual scale.  matvec = base + residual."""

    kind = HK_BIN_RICE

    def __init__(self, ctx: Context, rows: int, cols: int, bin_scales: np.ndarray, bin_signs: np.ndarray,
                 first_index: int, rice_k: int, rice: np.ndarray, outlier_count: int, residual_scale_f16: int,
                 residual_signs: np.ndarray):
        arrs = [np.ascontiguousarray(a, dt) for a, dt in
                ((bin_scales, np.uint16), (bin_signs, np.uint8), (rice, np.uint8), (residual_signs, np.uint8))]
        bs, bg, rc, sg = arrs
        src = RiceQ1Src(rows=rows, cols=cols, bin_scales=_ptr(bs), bin_signs=_ptr(bg), first_index=first_index,
                        rice_k=rice_k, rice=_ptr(rc) if rc.size else None, rice_bytes=rc.size,
                        outlier_count=outlier_count, residual_scale_f16=residual_scale_f16,
                        residual_signs=_ptr(sg))
        self._upload_rice(ctx, src)

    @classmethod
    def from_device(cls, ctx: Context, src: RiceQ1Src) -> "RiceQ1Packed":
        """An organ from a body already in device memory (hk_pack_binary_rice's output)."""
        self = cls.__new__(cls)
        self._upload_rice(ctx, src)
        return self

    def _upload_rice(self, ctx: Context, src: RiceQ1Src) -> None:
        self.ctx = ctx
        h = C.c_void_p()
        ctx.call("hk_organ_upload_rice", C.byref(src), ctx.stream, C.byref(h))
        self.h = h
        self.rows, self.cols, self.group = int(src.rows), int(src.cols), 128
        self.outlier_count = int(src.outlier_count)
        sz = C.c_size_t()
        ctx.check("hk_organ_info", ctx.L.hk_organ_info(h, None, None, None, None, C.byref(sz)))
        self.packed_bytes = int(sz.value)

    def apply_residual_device(self, x: DeviceArray, y: DeviceArray, stream=None) -> None:
        """y += residual x (the outliers of each row in index order)."""
        self.ctx.call("hk_rice_apply", self.h, x.ptr, y.ptr, stream if stream is not None else self.ctx.stream)


def binary_rice_q1_matvec_f32(packed: RiceQ1Packed, x: np.ndarray) -> np.ndarray:
    """GPU counterpart of binary_rice_q1_matvec_f32 (q80_mixed_decode.rs:509-527)."""
    return packed.matvec(x)


def pack_binary_rice_device(ctx: Context, w: DeviceArray, rows: int, cols: int, ratio: float = 0.02):
    """pack_binary_rice_q1 on the device: returns (RiceQ1Src with device
    pointers, the device buffers keeping them alive)."""
    n = rows * cols
    count = max(1, min(n, int(np.ceil(n * ratio))))
    bufs = (ctx.empty(n // 128, np.uint16), ctx.empty(n // 8, np.uint8), ctx.empty((count + 7) // 8, np.uint8),
            ctx.empty(((n + 17 * count) // 8 + 64) // 4 * 4, np.uint8))
    out = RiceQ1Src()
    ctx.call("hk_pack_binary_rice", w.ptr, rows, cols, ratio, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr,
             bufs[3].nbytes, C.byref(out), ctx.stream)
    return out, bufs


class MixedPackedTensor(PackedOrgan):
    """Per-128-group binary | Q2 organ from the canonical mixed stream."""

    kind = HK_MIXED

    def __init__(self, ctx: Context, rows: int, cols: int, tags: np.ndarray, bin_scales: np.ndarray,
                 bin_signs: np.ndarray, q2_scales: np.ndarray, q2_codes: np.ndarray):
        arrs = [np.ascontiguousarray(a, dt) for a, dt in
                ((tags, np.uint8), (bin_scales, np.uint16), (bin_signs, np.uint8),
                 (q2_scales, np.uint16), (q2_codes, np.uint8))]
        tags, bs, bg, qs, qc = arrs
        src = OrganSrc(kind=HK_MIXED, group=128, rows=rows, cols=cols, scales=_ptr(bs) if bs.size else None,
                       codes=_ptr(bg) if bg.size else None, tags=_ptr(tags),
                       q2_scales=_ptr(qs) if qs.size else None, q2_codes=_ptr(qc) if qc.size else None,
                       n_bin=bs.size, n_q2=qs.size // 2)
        super().__init__(ctx, src, tuple(arrs))


class DenseF32Organ(PackedOrgan):
    kind = HK_F32

    def __init__(self, ctx: Context, w: np.ndarray):
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = w.shape
        src = OrganSrc(kind=HK_F32, group=0, rows=rows, cols=cols, dense=_ptr(w))
        super().__init__(ctx, src, (w,))


class SyntheticOrgan(PackedOrgan):
    """An organ generated and packed on the device from the synthetic
    generator (weights N(0, sigma) from `key`, mixed coins from `coin_key`)."""

    def __init__(self, ctx: Context, kind: int, rows: int, cols: int, key: int, coin_key: int = 0,
                 group: int = 128, sigma: float = 0.02):
        self.ctx = ctx
        self.kind = kind
        h = C.c_void_p()
        ctx.call("hk_organ_synthetic", kind, group, rows, cols, key, coin_key, sigma, ctx.stream, C.byref(h))
        self.h = h
        self.rows, self.cols, self.group = rows, cols, group
        sz = C.c_size_t()
        ctx.check("hk_organ_info", ctx.L.hk_organ_info(h, None, None, None, None, C.byref(sz)))
        self.packed_bytes = int(sz.value)


class OrganSet:
    """Organs of one kind and shape with a device-resident descriptor table:
    `gemv` runs y_i = W_i x_i for all of them in one launch, no host sync."""

    def __init__(self, ctx: Context, organs: list[PackedOrgan]):
        self.ctx, self.organs = ctx, list(organs)
        arr = (C.c_void_p * len(organs))(*[o.h.value for o in organs])
        h = C.c_void_p()
        ctx.call("hk_organ_set_create", arr, len(organs), C.byref(h))
        self.h = h
        self.rows, self.cols = organs[0].rows, organs[0].cols

    def gemv(self, x: DeviceArray, x_stride: int, y: DeviceArray, y_stride: int, stream=None) -> None:
        self.ctx.call("hk_gemv_set", self.h, x.ptr, x_stride, y.ptr, y_stride,
                      stream if stream is not None else self.ctx.stream)

    @property
    def packed_bytes(self) -> int:
        return sum(o.packed_bytes for o in self.organs)

    def free(self):
        if getattr(self, "h", None) and self.h.value and self.ctx.h:
            self.ctx.L.hk_organ_set_free(self.ctx.h, self.h)
        self.h = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def gemv_lowrank_set(ctx: Context, lefts: OrganSet, rights: OrganSet, x: DeviceArray, x_stride: int,
                     y: DeviceArray, y_stride: int, stream=None, mid: DeviceArray | None = None,
                     mid_stride: int = 0) -> None:
    """y_i = L_i (R_i x_i) over the HGRAVS01 pairs of two organ sets
    (hk_gemv_lowrank_set): one launch for the shapes the fused kernel takes,
    else two through `mid` (n x rank floats, required then); mid, when given,
    receives R_i x_i."""
    ctx.call("hk_gemv_lowrank_set", lefts.h, rights.h, x.ptr, x_stride, mid.ptr if mid is not None else None,
             mid_stride, y.ptr, y_stride, stream if stream is not None else ctx.stream)


def gemv_batch(ctx: Context, organs: list[PackedOrgan], x: DeviceArray, x_stride: int, y: DeviceArray,
               y_stride: int, stream=None) -> None:
    """y_i = W_i x_i for organs of one kind and shape, in one launch
    (hk_gemv_batch: a synchronous helper that builds and frees a transient
    organ set; stream-ordered callers keep an OrganSet)."""
    arr = (C.c_void_p * len(organs))(*[o.h.value for o in organs])
    ctx.call("hk_gemv_batch", arr, len(organs), x.ptr, x_stride, y.ptr, y_stride,
             stream if stream is not None else ctx.stream)


# ---------------------------------------------------------------- device packers / generator

def pack_q4_device(ctx: Context, w: DeviceArray, rows: int, cols: int, group: int):
    scales = ctx.empty(rows * cols // group, np.uint16)
    codes = ctx.empty(rows * cols // 2, np.uint8)
    ctx.call("hk_pack_q4", w.ptr, rows, cols, group, scales.ptr, codes.ptr, ctx.stream)
    return scales, codes


def pack_binary_group_device(ctx: Context, w: DeviceArray, rows: int, cols: int):
    scales = ctx.empty(rows * cols // 128, np.uint16)
    signs = ctx.empty(rows * cols // 8, np.uint8)
    ctx.call("hk_pack_bin", w.ptr, rows, cols, scales.ptr, signs.ptr, ctx.stream)
    return scales, signs


def pack_q8_device(ctx: Context, w: DeviceArray, rows: int, cols: int):
    scales = ctx.empty(rows * cols // 64, np.uint16)
    codes = ctx.empty(rows * cols, np.uint8)
    ctx.call("hk_pack_q8", w.ptr, rows, cols, scales.ptr, codes.ptr, ctx.stream)
    return scales, codes


def pack_u3_device(ctx: Context, w: DeviceArray, count: int):
    groups = (count + 63) // 64
    scales = ctx.empty(groups, np.uint16)
    codes = ctx.empty(groups * 24, np.uint8)
    ctx.call("hk_pack_u3", w.ptr, count, scales.ptr, codes.ptr, ctx.stream)
    return scales, codes


def pack_q2_device(ctx: Context, w: DeviceArray, count: int):
    scales = ctx.empty(count // 64, np.uint16)
    codes = ctx.empty(count // 4, np.uint8)
    ctx.call("hk_pack_q2", w.ptr, count, scales.ptr, codes.ptr, ctx.stream)
    return scales, codes


def pack_mixed_device(ctx: Context, w: DeviceArray, rows: int, cols: int, is_binary: DeviceArray):
    """The per-group mixed packer on device buffers (hk_pack_mixed): returns
    the canonical stream (tags, bin_scales, bin_signs, q2_scales, q2_codes)
    as device arrays sized for the selector."""
    groups = rows * cols // 128
    sel = is_binary.download() if isinstance(is_binary, DeviceArray) else np.asarray(is_binary)
    nb = int(np.count_nonzero(sel))
    nq = groups - nb
    tags = ctx.empty((groups + 7) // 8, np.uint8)
    bs, bg = ctx.empty(max(nb, 1), np.uint16), ctx.empty(max(nb, 1) * 16, np.uint8)
    qs, qc = ctx.empty(max(nq, 1) * 2, np.uint16), ctx.empty(max(nq, 1) * 32, np.uint8)
    n_bin = C.c_uint32()
    sd = is_binary if isinstance(is_binary, DeviceArray) else ctx.to_device(np.ascontiguousarray(sel, np.uint8))
    ctx.call("hk_pack_mixed", w.ptr, rows, cols, sd.ptr, tags.ptr, bs.ptr, bg.ptr, nb, qs.ptr, qc.ptr, nq,
             C.byref(n_bin), ctx.stream)
    assert n_bin.value == nb
    return tags, bs, bg, qs, qc


def stream_key(seed: int, stream_id: int) -> int:
    return int(_lib.lib().hk_stream_key(seed, stream_id))


def synth_normal(ctx: Context, key: int, count: int, sigma: float, first: int = 0) -> DeviceArray:
    out = ctx.empty(count)
    ctx.call("hk_synth_normal", key, first, count, sigma, out.ptr, ctx.stream)
    return out
