"""ctypes view of the CPU oracle (oracle/hk_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker or the timed CPU
baseline, never by the product package (hawking_amd/).

Every function is a thin numpy wrapper over the C restatement; the C file
cites the reference function each one follows.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# HKO_ORACLE_LIB selects another build of the same sources (the sanitizer
# build that tests/test_sanitize.py runs the oracle tests against)
LIB_PATH = os.environ.get("HKO_ORACLE_LIB") or os.path.join(_HERE, "build", "libhk_oracle.so")

HKO_OK = 0

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_p = C.c_void_p
_sz = C.c_size_t


def _declare(L: C.CDLL) -> None:
    sig = {
        "hko_f32_to_f16": (C.c_uint16, [C.c_float]),
        "hko_f16_to_f32": (C.c_float, [C.c_uint16]),
        "hko_rint_ties_even": (C.c_float, [C.c_float]),
        "hko_deterministic_matrix": (None, [_sz, _sz, C.c_uint32, _p]),
        "hko_deterministic_input": (None, [_sz, _p]),
        "hko_stream_key": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "hko_normal": (C.c_float, [C.c_uint64, C.c_uint64, C.c_float]),
        "hko_fill_normal": (None, [C.c_uint64, _sz, C.c_float, _p]),
        "hko_fill_normal_from": (None, [C.c_uint64, C.c_uint64, _sz, C.c_float, _p]),
        "hko_mixed_coin": (C.c_int, [C.c_uint64, C.c_uint64]),
        "hko_fill_coins": (None, [C.c_uint64, _sz, _p]),
        "hko_q4_pack": (C.c_int, [_p, _sz, _sz, C.c_int, _p, _p]),
        "hko_q4_decode": (C.c_int, [_p, _p, _sz, _sz, C.c_int, _p]),
        "hko_q4_matvec": (C.c_int, [_p, _p, _sz, _sz, C.c_int, _p, _p]),
        "hko_q4_matvec_f64": (C.c_int, [_p, _p, _sz, _sz, C.c_int, _p, _p]),
        "hko_q4_0_dequant": (C.c_int, [_p, _sz, _p]),
        "hko_bin_pack": (C.c_int, [_p, _sz, _sz, C.c_int, _p, _p]),
        "hko_bin_decode": (C.c_int, [_p, _p, _sz, _sz, C.c_int, _p]),
        "hko_bin_matvec": (C.c_int, [_p, _p, _sz, _sz, C.c_int, _p, _p]),
        "hko_bin_matvec_f64": (C.c_int, [_p, _p, _sz, _sz, C.c_int, _p, _p]),
        "hko_q2_pack": (C.c_int, [_p, _sz, _p, _p]),
        "hko_q2_decode": (C.c_int, [_p, _p, _sz, _p]),
        "hko_uniform_packed_bytes": (_sz, [_sz, _sz, C.c_int, _sz]),
        "hko_uniform_pack": (C.c_int, [_p, _sz, _sz, C.c_int, _sz, _p, _p]),
        "hko_uniform_decode": (C.c_int, [_p, _p, _sz, _sz, C.c_int, _sz, _p]),
        "hko_uniform_matvec": (C.c_int, [_p, _p, _sz, _sz, C.c_int, _sz, _p, _p]),
        "hko_uniform_matvec_f64": (C.c_int, [_p, _p, _sz, _sz, C.c_int, _sz, _p, _p]),
        "hko_hgravs01_matvec": (C.c_int, [_p, _p, _sz, _sz, _p, _p, _sz, C.c_int, _sz, _p, _p]),
        "hko_best_rice_k": (C.c_uint32, [_p, _sz]),
        "hko_rice_bytes": (_sz, [_p, _sz, C.c_uint32]),
        "hko_rice_pack": (None, [_p, _sz, C.c_uint32, _p]),
        "hko_rice_unpack": (C.c_int, [_p, _sz, _sz, C.c_uint32, _p]),
        "hko_rice_expand": (C.c_int, [C.c_uint32, _p, _sz, C.c_uint32, _sz, _p]),
        "hko_rice_row_ptr": (C.c_int, [_p, _sz, _sz, _sz, _p]),
        "hko_rice_q1_count": (_sz, [_sz, C.c_double]),
        "hko_rice_q1_pack": (C.c_int, [_p, _sz, _sz, C.c_double, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
        "hko_rice_q1_apply": (C.c_int, [_p, _p, _sz, C.c_uint16, _sz, _sz, _p, _p]),
        "hko_rice_q1_matvec": (C.c_int, [_p, _p, _sz, _sz, _p, _p, _sz, C.c_uint16, _p, _p]),
        "hko_rice_q1_matvec_f64": (C.c_int, [_p, _p, _sz, _sz, _p, _p, _sz, C.c_uint16, _p, _p]),
        "hko_mixed_pack": (C.c_int, [_p, _sz, _sz, _p, _p]),
        "hko_mixed_free": (None, [_p]),
        "hko_mixed_decode": (C.c_int, [_p, _p]),
        "hko_mixed_matvec": (C.c_int, [_p, _p, _p]),
        "hko_mixed_matvec_f64": (C.c_int, [_p, _p, _p]),
        "hko_gemv_f32": (None, [_p, _sz, _sz, _p, _p]),
        "hko_router_softmax_topk": (C.c_int, [_p, _sz, _sz, C.c_float, _p, _p]),
        "hko_topk_softmax_batch": (None, [_p, _sz, _sz, _sz, _p, _p]),
        "hko_router_noaux_tc": (C.c_int, [_p, _p, _sz, _sz, _sz, _sz, C.c_int, C.c_float, _p, _p]),
        "hko_topk_desc": (None, [_p, _sz, _sz, _p]),
        "hko_rmsnorm_1p": (C.c_int, [_p, _p, _sz, C.c_float, _p]),
        "hko_silu_mul": (None, [_p, _p, _sz, _p]),
        "hko_argmax_greedy": (C.c_int, [_p, _sz, _p]),
        "hko_terminal_greedy": (C.c_int, [_p, _p, _sz, C.c_float, _p, _p, _sz, _sz, _p, _p]),
        "hko_organ_matvec": (C.c_int, [_p, _p, _p]),
        "hko_mlp": (C.c_int, [_p, _p, _p, _p, _p, _p]),
        "hko_moe_layer_forward": (C.c_int, [_p, _p, _p, _p, _p, _p, _p]),
        "hko_moe_layer_forward_f64": (C.c_int, [_p, _p, _p, _p, _p]),
        "hko_noaux_moe_forward": (C.c_int, [_p, _p, _p, _p, _p, _p]),
        "hko_noaux_moe_forward_f64": (C.c_int, [_p, _p, _p, _p]),
        "hko_relative_l2_f32": (C.c_double, [_p, _p, _sz]),
        "hko_relative_l2_f64ref": (C.c_double, [_p, _p, _sz]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


class OracleError(RuntimeError):
    def __init__(self, fn: str, code: int):
        super().__init__(f"{fn} returned status {code}")
        self.code = code


def _check(fn: str, rc: int) -> None:
    if rc != HKO_OK:
        raise OracleError(fn, rc)


# ---- scalars -------------------------------------------------------------

def f32_to_f16(v: float) -> int:
    return lib().hko_f32_to_f16(float(v))


def f16_to_f32(bits: int) -> float:
    return lib().hko_f16_to_f32(int(bits))


def rint_ties_even(v: float) -> float:
    return lib().hko_rint_ties_even(float(v))


# ---- generators ------------------------------------------------------------

def deterministic_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    out = np.empty(rows * cols, np.float32)
    lib().hko_deterministic_matrix(rows, cols, seed, _ptr(out))
    return out.reshape(rows, cols)


def deterministic_input(cols: int) -> np.ndarray:
    out = np.empty(cols, np.float32)
    lib().hko_deterministic_input(cols, _ptr(out))
    return out


def stream_key(seed: int, stream: int) -> int:
    return lib().hko_stream_key(seed, stream)


def normal(key: int, count: int, sigma: float, first: int = 0) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().hko_fill_normal_from(key, first, count, sigma, _ptr(out))
    return out


def mixed_coins(coin_key: int, groups: int) -> np.ndarray:
    out = np.empty(groups, np.uint8)
    lib().hko_fill_coins(coin_key, groups, _ptr(out))
    return out


# ---- Q4 ------------------------------------------------------------------------

def q4_pack(w: np.ndarray, group: int):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    groups = rows * cols // max(group, 1)
    scales = np.zeros(max(groups, 1), np.uint16)
    codes = np.zeros(max(rows * cols // 2, 1), np.uint8)
    _check("hko_q4_pack", lib().hko_q4_pack(_ptr(w), rows, cols, group, _ptr(scales), _ptr(codes)))
    return scales, codes


def q4_decode(scales, codes, rows, cols, group) -> np.ndarray:
    out = np.empty(rows * cols, np.float32)
    _check("hko_q4_decode", lib().hko_q4_decode(_ptr(scales), _ptr(codes), rows, cols, group, _ptr(out)))
    return out.reshape(rows, cols)


def q4_matvec(scales, codes, rows, cols, group, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    _check("hko_q4_matvec",
           lib().hko_q4_matvec(_ptr(scales), _ptr(codes), rows, cols, group, _ptr(x), _ptr(y)))
    return y


def q4_matvec_f64(scales, codes, rows, cols, group, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float64)
    y = np.empty(rows, np.float64)
    _check("hko_q4_matvec_f64",
           lib().hko_q4_matvec_f64(_ptr(scales), _ptr(codes), rows, cols, group, _ptr(x), _ptr(y)))
    return y


def q4_0_dequant(blocks: np.ndarray, elements: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8)
    out = np.empty(elements, np.float32)
    _check("hko_q4_0_dequant", lib().hko_q4_0_dequant(_ptr(blocks), elements, _ptr(out)))
    return out


# ---- binary ----------------------------------------------------------------------

def bin_pack(w: np.ndarray, group: int = 128):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    scales = np.zeros(rows * cols // group, np.uint16)
    signs = np.zeros((rows * cols + 7) // 8, np.uint8)
    _check("hko_bin_pack", lib().hko_bin_pack(_ptr(w), rows, cols, group, _ptr(scales), _ptr(signs)))
    return scales, signs


def bin_decode(scales, signs, rows, cols, group=128) -> np.ndarray:
    out = np.empty(rows * cols, np.float32)
    _check("hko_bin_decode", lib().hko_bin_decode(_ptr(scales), _ptr(signs), rows, cols, group, _ptr(out)))
    return out.reshape(rows, cols)


def bin_matvec(scales, signs, rows, cols, x, group=128) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    _check("hko_bin_matvec",
           lib().hko_bin_matvec(_ptr(scales), _ptr(signs), rows, cols, group, _ptr(x), _ptr(y)))
    return y


def bin_matvec_f64(scales, signs, rows, cols, x, group=128) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float64)
    y = np.empty(rows, np.float64)
    _check("hko_bin_matvec_f64",
           lib().hko_bin_matvec_f64(_ptr(scales), _ptr(signs), rows, cols, group, _ptr(x), _ptr(y)))
    return y


# ---- Q2 / mixed ------------------------------------------------------------------

def q2_pack(w: np.ndarray):
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    scales = np.zeros(w.size // 64, np.uint16)
    codes = np.zeros(w.size // 4, np.uint8)
    _check("hko_q2_pack", lib().hko_q2_pack(_ptr(w), w.size, _ptr(scales), _ptr(codes)))
    return scales, codes


def q2_decode(scales, codes, count) -> np.ndarray:
    out = np.empty(count, np.float32)
    _check("hko_q2_decode", lib().hko_q2_decode(_ptr(scales), _ptr(codes), count, _ptr(out)))
    return out


# ---- uniform factor codec (HGRAVU01 q8 G64, HGRAVS01 factors) -------------------

def uniform_pack(w: np.ndarray, rows: int, cols: int, bits: int = 8, group: int = 64):
    """pack_uniform_factor: (scales f16 bits [groups], packed codes)."""
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    assert w.size == rows * cols
    groups = -(-rows * cols // group)
    scales = np.zeros(groups, np.uint16)
    codes = np.zeros(lib().hko_uniform_packed_bytes(rows, cols, bits, group), np.uint8)
    _check("hko_uniform_pack", lib().hko_uniform_pack(_ptr(w), rows, cols, bits, group, _ptr(scales), _ptr(codes)))
    return scales, codes


def uniform_decode(scales, codes, rows, cols, bits=8, group=64) -> np.ndarray:
    out = np.empty(rows * cols, np.float32)
    _check("hko_uniform_decode",
           lib().hko_uniform_decode(_ptr(scales), _ptr(codes), rows, cols, bits, group, _ptr(out)))
    return out.reshape(rows, cols)


def uniform_matvec(scales, codes, rows, cols, x, bits=8, group=64) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    _check("hko_uniform_matvec",
           lib().hko_uniform_matvec(_ptr(scales), _ptr(codes), rows, cols, bits, group, _ptr(x), _ptr(y)))
    return y


def uniform_matvec_f64(scales, codes, rows, cols, x, bits=8, group=64) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float64)
    y = np.empty(rows, np.float64)
    _check("hko_uniform_matvec_f64",
           lib().hko_uniform_matvec_f64(_ptr(scales), _ptr(codes), rows, cols, bits, group, _ptr(x), _ptr(y)))
    return y


def hgravs01_matvec(left, right, rows, rank, cols, x, bits=3, group=64) -> np.ndarray:
    """hgravs01_two_stage_matvec_f32: y = L (R x); left/right = (scales, codes)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    _check("hko_hgravs01_matvec",
           lib().hko_hgravs01_matvec(_ptr(left[0]), _ptr(left[1]), rows, rank, _ptr(right[0]), _ptr(right[1]),
                                     cols, bits, group, _ptr(x), _ptr(y)))
    return y


# ---- HGRAVR02 binary + Rice-coded 1-bit residual (rice_q1_rms) ------------------

def best_rice_k(values) -> int:
    v = np.ascontiguousarray(values, np.uint32)
    return int(lib().hko_best_rice_k(_ptr(v), v.size))


def rice_pack(values, k: int) -> np.ndarray:
    v = np.ascontiguousarray(values, np.uint32)
    out = np.zeros(lib().hko_rice_bytes(_ptr(v), v.size, k), np.uint8)
    lib().hko_rice_pack(_ptr(v), v.size, k, _ptr(out))
    return out


def rice_unpack(payload, count: int, k: int) -> np.ndarray:
    p = np.ascontiguousarray(payload, np.uint8)
    out = np.zeros(max(count, 1), np.uint32)
    _check("hko_rice_unpack", lib().hko_rice_unpack(_ptr(p), p.size, count, k, _ptr(out)))
    return out[:count]


def rice_expand(first: int, rice, k: int, count: int) -> np.ndarray:
    p = np.ascontiguousarray(rice, np.uint8)
    out = np.zeros(max(count, 1), np.uint32)
    _check("hko_rice_expand", lib().hko_rice_expand(first, _ptr(p) if p.size else None, p.size, k, count, _ptr(out)))
    return out[:count]


def rice_row_ptr(indices, rows: int, cols: int) -> np.ndarray:
    i = np.ascontiguousarray(indices, np.uint32)
    out = np.zeros(rows + 1, np.uint32)
    _check("hko_rice_row_ptr", lib().hko_rice_row_ptr(_ptr(i), i.size, rows, cols, _ptr(out)))
    return out


@dataclass
class RiceQ1:
    """pack_binary_rice_q1's RiceQ1Packed: the binary body, the outliers'
    flat indices, their sign bits, the f16 RMS scale, and the Rice stream."""
    rows: int
    cols: int
    bin_scales: np.ndarray
    bin_signs: np.ndarray
    indices: np.ndarray
    res_signs: np.ndarray
    res_scale: int
    first: int
    rice_k: int
    rice: np.ndarray

    @property
    def count(self) -> int:
        return int(self.indices.size)


def rice_q1_pack(w: np.ndarray, rows: int, cols: int, ratio: float = 0.02) -> RiceQ1:
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    assert w.size == rows * cols
    n = rows * cols
    count = int(lib().hko_rice_q1_count(n, ratio))
    bs = np.zeros(max(n // 128, 1), np.uint16)
    bg = np.zeros((n + 7) // 8, np.uint8)
    idx = np.zeros(count, np.uint32)
    sg = np.zeros((count + 7) // 8, np.uint8)
    cap = (n + 17 * count) // 8 + 1
    rice = np.zeros(cap, np.uint8)
    sc, first, k, ln = C.c_uint16(), C.c_uint32(), C.c_uint32(), C.c_size_t()
    _check("hko_rice_q1_pack",
           lib().hko_rice_q1_pack(_ptr(w), rows, cols, ratio, _ptr(bs), _ptr(bg), _ptr(idx), _ptr(sg), C.byref(sc),
                                  C.byref(first), C.byref(k), _ptr(rice), cap, C.byref(ln)))
    return RiceQ1(rows, cols, bs, bg, idx, sg, int(sc.value), int(first.value), int(k.value),
                  rice[:ln.value].copy())


def rice_q1_apply(p: RiceQ1, x, y0) -> np.ndarray:
    """y0 + the residual corrections in index order (the residual half of
    binary_rice_q1_matvec_f32)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.array(y0, np.float32, copy=True)
    _check("hko_rice_q1_apply", lib().hko_rice_q1_apply(_ptr(p.indices), _ptr(p.res_signs), p.count, p.res_scale,
                                                        p.rows, p.cols, _ptr(x), _ptr(y)))
    return y


def rice_q1_matvec(p: RiceQ1, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(p.rows, np.float32)
    _check("hko_rice_q1_matvec",
           lib().hko_rice_q1_matvec(_ptr(p.bin_scales), _ptr(p.bin_signs), p.rows, p.cols, _ptr(p.indices),
                                    _ptr(p.res_signs), p.count, p.res_scale, _ptr(x), _ptr(y)))
    return y


def rice_q1_matvec_f64(p: RiceQ1, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float64)
    y = np.empty(p.rows, np.float64)
    _check("hko_rice_q1_matvec_f64",
           lib().hko_rice_q1_matvec_f64(_ptr(p.bin_scales), _ptr(p.bin_signs), p.rows, p.cols, _ptr(p.indices),
                                        _ptr(p.res_signs), p.count, p.res_scale, _ptr(x), _ptr(y)))
    return y


class _Mixed(C.Structure):
    _fields_ = [
        ("rows", _sz), ("cols", _sz), ("n_bin", _sz), ("n_q2", _sz),
        ("tags", C.POINTER(C.c_uint8)), ("bin_scales", C.POINTER(C.c_uint16)),
        ("bin_signs", C.POINTER(C.c_uint8)), ("q2_scales", C.POINTER(C.c_uint16)),
        ("q2_codes", C.POINTER(C.c_uint8)),
    ]


@dataclass
class MixedPacked:
    """Canonical mixed stream (numpy copies) plus the live C struct."""
    rows: int
    cols: int
    tags: np.ndarray
    bin_scales: np.ndarray
    bin_signs: np.ndarray
    q2_scales: np.ndarray
    q2_codes: np.ndarray
    _c: _Mixed

    @property
    def n_bin(self) -> int:
        return int(self.bin_scales.size)

    @property
    def n_q2(self) -> int:
        return int(self.q2_scales.size // 2)

    def nbytes(self) -> int:
        return int(self.tags.nbytes + self.bin_scales.nbytes + self.bin_signs.nbytes
                   + self.q2_scales.nbytes + self.q2_codes.nbytes)

    def __del__(self):
        try:
            lib().hko_mixed_free(C.byref(self._c))
        except Exception:
            pass


def mixed_pack(w: np.ndarray, is_binary: np.ndarray) -> MixedPacked:
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    sel = np.ascontiguousarray(is_binary, np.uint8)
    m = _Mixed()
    _check("hko_mixed_pack", lib().hko_mixed_pack(_ptr(w), rows, cols, _ptr(sel), C.byref(m)))
    groups = rows * cols // 128

    def arr(p, n, dt):
        return np.ctypeslib.as_array(p, shape=(n,)).astype(dt, copy=True) if n else np.zeros(0, dt)

    return MixedPacked(
        rows, cols,
        arr(m.tags, (groups + 7) // 8, np.uint8),
        arr(m.bin_scales, m.n_bin, np.uint16),
        arr(m.bin_signs, m.n_bin * 16, np.uint8),
        arr(m.q2_scales, m.n_q2 * 2, np.uint16),
        arr(m.q2_codes, m.n_q2 * 32, np.uint8),
        m,
    )


def mixed_decode(m: MixedPacked) -> np.ndarray:
    out = np.empty(m.rows * m.cols, np.float32)
    _check("hko_mixed_decode", lib().hko_mixed_decode(C.byref(m._c), _ptr(out)))
    return out.reshape(m.rows, m.cols)


def mixed_matvec(m: MixedPacked, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(m.rows, np.float32)
    _check("hko_mixed_matvec", lib().hko_mixed_matvec(C.byref(m._c), _ptr(x), _ptr(y)))
    return y


def mixed_matvec_f64(m: MixedPacked, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float64)
    y = np.empty(m.rows, np.float64)
    _check("hko_mixed_matvec_f64", lib().hko_mixed_matvec_f64(C.byref(m._c), _ptr(x), _ptr(y)))
    return y


# ---- dense / router / activations ------------------------------------------------

def gemv_f32(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(w.shape[0], np.float32)
    lib().hko_gemv_f32(_ptr(w), w.shape[0], w.shape[1], _ptr(x), _ptr(y))
    return y


def router_softmax_topk(logits, top_k, tie_eps=0.0):
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(top_k, np.int32)
    wts = np.empty(top_k, np.float32)
    _check("hko_router_softmax_topk",
           lib().hko_router_softmax_topk(_ptr(logits), logits.size, top_k, tie_eps, _ptr(ids), _ptr(wts)))
    return ids, wts


def topk_softmax_batch(logits, n_tokens, n_experts, top_k):
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(n_tokens * top_k, np.int32)
    wts = np.empty(n_tokens * top_k, np.float32)
    lib().hko_topk_softmax_batch(_ptr(logits), n_tokens, n_experts, top_k, _ptr(ids), _ptr(wts))
    return ids, wts


def router_noaux_tc(logits, bias, n_group, topk_group, top_k, norm_topk_prob=True, scaling=1.0):
    logits = np.ascontiguousarray(logits, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    ids = np.empty(top_k, np.int32)
    wts = np.empty(top_k, np.float32)
    _check("hko_router_noaux_tc",
           lib().hko_router_noaux_tc(_ptr(logits), _ptr(bias), logits.size, n_group, topk_group,
                                     top_k, int(norm_topk_prob), scaling, _ptr(ids), _ptr(wts)))
    return ids, wts


def topk_desc(values, k):
    values = np.ascontiguousarray(values, np.float32)
    out = np.empty(min(k, values.size), np.int32)
    lib().hko_topk_desc(_ptr(values), values.size, k, _ptr(out))
    return out


def rmsnorm_1p(x, w, eps=1e-6):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    _check("hko_rmsnorm_1p", lib().hko_rmsnorm_1p(_ptr(x), _ptr(w), x.size, eps, _ptr(out)))
    return out


def silu_mul(g, u):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    lib().hko_silu_mul(_ptr(g), _ptr(u), g.size, _ptr(out))
    return out


def relative_l2(candidate, reference) -> float:
    c = np.ascontiguousarray(candidate, np.float32).reshape(-1)
    if np.asarray(reference).dtype == np.float64:
        r = np.ascontiguousarray(reference, np.float64).reshape(-1)
        return lib().hko_relative_l2_f64ref(_ptr(c), _ptr(r), c.size)
    r = np.ascontiguousarray(reference, np.float32).reshape(-1)
    return lib().hko_relative_l2_f32(_ptr(c), _ptr(r), c.size)


# ---- organs and the MoE layer ----------------------------------------------------------

class _Organ(C.Structure):
    _fields_ = [
        ("kind", C.c_int), ("group", C.c_int), ("rows", _sz), ("cols", _sz),
        ("scales", _p), ("codes", _p), ("mixed", _p),
        ("rank", _sz), ("r_scales", _p), ("r_codes", _p),
        ("res_indices", _p), ("res_signs", _p), ("res_count", _sz), ("res_scale", C.c_uint16),
    ]


class Organ:
    """One packed matrix for the oracle: kind 0 = Q4, 1 = binary, 2 = mixed,
    3 = uniform q8 G64, 4 = low-rank 3-bit factors, 5 = binary + Rice residual."""

    def __init__(self, kind, rows, cols, group=0, scales=None, codes=None, mixed=None, rank=0, right=None,
                 rice=None):
        self.kind, self.rows, self.cols, self.group = kind, rows, cols, group
        self.scales, self.codes, self.mixed, self.rank, self.right, self.rice = scales, codes, mixed, rank, right, rice
        self.c = _Organ(kind, group, rows, cols, _ptr(scales), _ptr(codes),
                        C.cast(C.byref(mixed._c), _p) if mixed is not None else None, rank,
                        _ptr(right[0]) if right is not None else None, _ptr(right[1]) if right is not None else None,
                        _ptr(rice.indices) if rice is not None else None,
                        _ptr(rice.res_signs) if rice is not None else None,
                        rice.count if rice is not None else 0, rice.res_scale if rice is not None else 0)

    @classmethod
    def uniform8(cls, w):
        s, c = uniform_pack(w, w.shape[0], w.shape[1], 8, 64)
        return cls(3, w.shape[0], w.shape[1], 64, s, c)

    @classmethod
    def low_rank(cls, left_w, right_w):
        """HGRAVS01 from its two factors (3-bit G64)."""
        rows, rank = left_w.shape
        cols = right_w.shape[1]
        ls, lc = uniform_pack(left_w, rows, rank, 3, 64)
        rs, rc = uniform_pack(right_w, rank, cols, 3, 64)
        return cls(4, rows, cols, 64, ls, lc, rank=rank, right=(rs, rc))

    @classmethod
    def rice_q1(cls, w, ratio=0.02):
        p = rice_q1_pack(w, w.shape[0], w.shape[1], ratio)
        return cls(5, w.shape[0], w.shape[1], 128, p.bin_scales, p.bin_signs, rice=p)

    @classmethod
    def q4(cls, w, group):
        s, c = q4_pack(w, group)
        return cls(0, w.shape[0], w.shape[1], group, s, c)

    @classmethod
    def binary(cls, w):
        s, c = bin_pack(w, 128)
        return cls(1, w.shape[0], w.shape[1], 128, s, c)

    @classmethod
    def mixed_from(cls, w, is_binary):
        m = mixed_pack(w, is_binary)
        return cls(2, w.shape[0], w.shape[1], 128, mixed=m)

    def matvec(self, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(self.rows, np.float32)
        _check("hko_organ_matvec", lib().hko_organ_matvec(C.byref(self.c), _ptr(x), _ptr(y)))
        return y


class _MoeLayer(C.Structure):
    _fields_ = [
        ("hidden", _sz), ("inter", _sz), ("n_experts", _sz), ("top_k", _sz), ("eps", C.c_float),
        ("norm_w", _p), ("router_w", _p), ("shared_gate_w", _p), ("experts", _p), ("shared", _p),
        ("tie_eps", C.c_float),
    ]


class MoeLayer:
    """Oracle view of one moe_suffix layer.  experts: list of (gate, up, down) Organs
    indexed by expert id; entries may be None for experts the caller knows are unused
    (the oracle touches only the routed ids)."""

    def __init__(self, hidden, inter, n_experts, top_k, norm_w, router_w, experts,
                 shared=None, shared_gate_w=None, eps=1e-6, tie_eps=0.0):
        self.norm_w = np.ascontiguousarray(norm_w, np.float32)
        self.router_w = np.ascontiguousarray(router_w, np.float32)
        self.shared_gate_w = None if shared_gate_w is None else np.ascontiguousarray(shared_gate_w, np.float32)
        self._experts = experts
        self._shared = shared
        arr = (_Organ * (n_experts * 3))()
        for e, trip in enumerate(experts):
            if trip is None:
                continue
            for j in range(3):
                arr[e * 3 + j] = trip[j].c
        self._arr = arr
        sh = None
        if shared is not None:
            sh = (_Organ * 3)(shared[0].c, shared[1].c, shared[2].c)
        self._sh = sh
        self.c = _MoeLayer(hidden, inter, n_experts, top_k, eps, _ptr(self.norm_w),
                           _ptr(self.router_w), _ptr(self.shared_gate_w),
                           C.cast(arr, _p), C.cast(sh, _p) if sh is not None else None, tie_eps)
        self.hidden, self.n_experts, self.top_k = hidden, n_experts, top_k

    def forward(self, h):
        h = np.ascontiguousarray(h, np.float32)
        out = np.empty(self.hidden, np.float32)
        ids = np.empty(self.top_k, np.int32)
        wts = np.empty(self.top_k, np.float32)
        xn = np.empty(self.hidden, np.float32)
        logits = np.empty(self.n_experts, np.float32)
        _check("hko_moe_layer_forward",
               lib().hko_moe_layer_forward(C.byref(self.c), _ptr(h), _ptr(out), _ptr(ids), _ptr(wts),
                                           _ptr(xn), _ptr(logits)))
        return out, ids, wts, xn, logits

    def forward_f64(self, h, ids):
        h = np.ascontiguousarray(h, np.float64)
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty(self.hidden, np.float64)
        _check("hko_moe_layer_forward_f64",
               lib().hko_moe_layer_forward_f64(C.byref(self.c), _ptr(h), _ptr(ids), None, _ptr(out)))
        return out


class _NoauxMoe(C.Structure):
    _fields_ = [
        ("hidden", _sz), ("n_experts", _sz), ("top_k", _sz), ("n_group", _sz), ("topk_group", _sz),
        ("norm_topk_prob", C.c_int), ("routed_scaling_factor", C.c_float),
        ("router_w", _p), ("bias", _p), ("experts", _p), ("shared", _p),
    ]


class NoauxMoe:
    """Oracle view of one noaux_tc MoE block (gravity_glm.rs routed_moe).  experts:
    list of (gate, up, down) Organs indexed by expert id; entries may be None for
    experts the caller knows are unused."""

    def __init__(self, hidden, n_experts, top_k, n_group, topk_group, norm_topk_prob, scaling,
                 router_w, bias, experts, shared=None):
        self.router_w = np.ascontiguousarray(router_w, np.float32)
        self.bias = np.ascontiguousarray(bias, np.float32)
        self._experts, self._shared = experts, shared
        arr = (_Organ * (n_experts * 3))()
        for e, trip in enumerate(experts):
            if trip is None:
                continue
            for j in range(3):
                arr[e * 3 + j] = trip[j].c
        self._arr = arr
        sh = (_Organ * 3)(shared[0].c, shared[1].c, shared[2].c) if shared is not None else None
        self._sh = sh
        self.c = _NoauxMoe(hidden, n_experts, top_k, n_group, topk_group, int(norm_topk_prob), scaling,
                           _ptr(self.router_w), _ptr(self.bias), C.cast(arr, _p),
                           C.cast(sh, _p) if sh is not None else None)
        self.hidden, self.n_experts, self.top_k = hidden, n_experts, top_k

    def forward(self, x):
        """Returns (out, ids, weights, logits) for one token."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(self.hidden, np.float32)
        ids = np.empty(self.top_k, np.int32)
        wts = np.empty(self.top_k, np.float32)
        logits = np.empty(self.n_experts, np.float32)
        _check("hko_noaux_moe_forward",
               lib().hko_noaux_moe_forward(C.byref(self.c), _ptr(x), _ptr(out), _ptr(ids), _ptr(wts), _ptr(logits)))
        return out, ids, wts, logits

    def forward_f64(self, x, ids):
        x = np.ascontiguousarray(x, np.float64)
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty(self.hidden, np.float64)
        _check("hko_noaux_moe_forward_f64",
               lib().hko_noaux_moe_forward_f64(C.byref(self.c), _ptr(x), _ptr(ids), _ptr(out)))
        return out


# ---- terminal head (final RMSNorm(1+w) -> lm_head q8 -> greedy argmax) ------------

def argmax_greedy(logits, n_valid: int | None = None) -> int:
    """terminal_greedy's pick: the lowest index of the largest non-NaN logit
    among the first n_valid; OracleError if that logit is not finite."""
    lg = np.ascontiguousarray(logits, np.float32)
    n = lg.size if n_valid is None else n_valid
    t = C.c_int32()
    _check("hko_argmax_greedy", lib().hko_argmax_greedy(_ptr(lg), n, C.byref(t)))
    return int(t.value)


def terminal_greedy(hidden, norm_w, scales, codes, vocab: int, n_valid: int, eps: float = 1e-6):
    """terminal_greedy with an HGRAVU01 lm_head: (token, logits)."""
    h = np.ascontiguousarray(hidden, np.float32)
    w = np.ascontiguousarray(norm_w, np.float32)
    logits = np.empty(vocab, np.float32)
    t = C.c_int32()
    _check("hko_terminal_greedy", lib().hko_terminal_greedy(_ptr(h), _ptr(w), h.size, eps, _ptr(scales), _ptr(codes),
                                                            vocab, n_valid, _ptr(logits), C.byref(t)))
    return int(t.value), logits
