"""ctypes binding of the C ABI in include/hawking_hip.h.

Loads hawking_amd/lib/libhawking_hip.so and nothing else: if the library is
missing or fails to load, every entry point raises.  There is no CPU path.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libhawking_hip.so")

HK_OK = 0
HK_E_INVALID_ARG = 1
HK_E_GEOMETRY = 2
HK_E_NONFINITE = 3
HK_E_HIP = 4
HK_E_UNSUPPORTED = 5
HK_E_ROUTE = 6
HK_E_NOMEM = 7

HK_Q4, HK_BIN, HK_MIXED, HK_F32, HK_Q8, HK_U3, HK_BIN_RICE = 0, 1, 2, 3, 4, 5, 6
HK_ROUTER_SOFTMAX, HK_ROUTER_NOAUX_TC = 0, 1
HK_STACK_PER_LAYER, HK_STACK_PERSISTENT = 0, 1

STATUS_NAMES = {
    HK_OK: "HK_OK", HK_E_INVALID_ARG: "HK_E_INVALID_ARG", HK_E_GEOMETRY: "HK_E_GEOMETRY",
    HK_E_NONFINITE: "HK_E_NONFINITE", HK_E_HIP: "HK_E_HIP", HK_E_UNSUPPORTED: "HK_E_UNSUPPORTED",
    HK_E_ROUTE: "HK_E_ROUTE", HK_E_NOMEM: "HK_E_NOMEM",
}

_p = C.c_void_p
_sz = C.c_size_t
_u32 = C.c_uint32
_i32 = C.c_int32
_u64 = C.c_uint64


class OrganSrc(C.Structure):
    _fields_ = [
        ("kind", _i32), ("group", _i32), ("rows", _u32), ("cols", _u32),
        ("scales", _p), ("codes", _p), ("tags", _p), ("q2_scales", _p), ("q2_codes", _p),
        ("n_bin", _u32), ("n_q2", _u32), ("dense", _p),
    ]


class RiceQ1Src(C.Structure):
    """hk_rice_q1: an HGRAVR02 body (host or device pointers)."""
    _fields_ = [
        ("rows", _u32), ("cols", _u32), ("bin_scales", _p), ("bin_signs", _p), ("first_index", _u32),
        ("rice_k", _u32), ("rice", _p), ("rice_bytes", _sz), ("outlier_count", _sz),
        ("residual_scale_f16", C.c_uint16), ("residual_signs", _p),
    ]


class CatalogRecord(C.Structure):
    """hk_catalog_record: one 128-byte HQ80M15 tensor record, decoded."""
    _fields_ = [
        ("name", C.c_char_p), ("codec", _u32), ("organ", _u32), ("ndim", _u32), ("shape", _u32 * 4),
        ("elements", _u64), ("segment_id", C.c_uint16), ("achieved_rank", C.c_uint16), ("offset", _u64),
        ("nbytes", _u64), ("sha256", C.c_uint8 * 32), ("flags", _u32), ("n_fit_rows", _u32),
        ("codec_bpw", C.c_float),
    ]


class MoeConfig(C.Structure):
    _fields_ = [
        ("n_layers", _u32), ("hidden", _u32), ("inter", _u32), ("shared_inter", _u32),
        ("n_experts", _u32), ("top_k", _u32), ("expert_kind", _i32), ("expert_group", _i32),
        ("shared_gate", _i32), ("eps", C.c_float), ("router", _i32), ("n_group", _u32), ("topk_group", _u32),
        ("norm_topk_prob", _i32), ("routed_scaling_factor", C.c_float), ("route_tie_eps", C.c_float),
        ("stack_launch", _i32),
    ]


class MoeLayerSrc(C.Structure):
    _fields_ = [
        ("norm_w", _p), ("router_w", _p), ("shared_gate_w", _p), ("experts", _p), ("shared", _p),
        ("router_bias", _p),
    ]


class Moe15LayerSrc(C.Structure):
    _fields_ = [
        ("hidden", _u32), ("inter", _u32), ("shared_inter", _u32), ("n_experts", _u32), ("top_k", _u32),
        ("eps", C.c_float), ("route_tie_eps", C.c_float), ("norm_w", _p), ("router", _p), ("shared_gate", _p), ("shared_gate_proj", _p),
        ("shared_up", _p), ("shared_down", _p), ("gate", _p), ("up", _p), ("down_left", _p), ("down_right", _p),
    ]


# name -> (restype, argtypes)
PROTOTYPES = {
    "hk_ctx_create": (C.c_int, [C.c_int, C.POINTER(_p)]),
    "hk_ctx_destroy": (None, [_p]),
    "hk_last_error": (C.c_int, [_p, C.c_char_p, _sz]),
    "hk_version": (C.c_char_p, []),
    "hk_device_info": (C.c_int, [_p, C.c_char_p, _sz, C.POINTER(C.c_int), C.POINTER(_sz)]),
    "hk_malloc": (C.c_int, [_p, _sz, C.POINTER(_p)]),
    "hk_free": (C.c_int, [_p, _p]),
    "hk_memcpy_htod": (C.c_int, [_p, _p, _p, _sz, _p]),
    "hk_memcpy_dtoh": (C.c_int, [_p, _p, _p, _sz, _p]),
    "hk_memcpy_dtod": (C.c_int, [_p, _p, _p, _sz, _p]),
    "hk_memset": (C.c_int, [_p, _p, C.c_int, _sz, _p]),
    "hk_stream_create": (C.c_int, [_p, C.POINTER(_p)]),
    "hk_stream_destroy": (C.c_int, [_p, _p]),
    "hk_stream_synchronize": (C.c_int, [_p, _p]),
    "hk_device_synchronize": (C.c_int, [_p]),
    "hk_event_create": (C.c_int, [_p, C.POINTER(_p)]),
    "hk_event_destroy": (C.c_int, [_p, _p]),
    "hk_event_record": (C.c_int, [_p, _p, _p]),
    "hk_event_elapsed_ms": (C.c_int, [_p, _p, _p, C.POINTER(C.c_float)]),
    "hk_check_device_status": (C.c_int, [_p, _p, C.POINTER(_u32)]),
    "hk_stream_control": (C.c_int, [_p, _p, _sz, _p, _u32, _p]),
    "hk_organ_upload": (C.c_int, [_p, C.POINTER(OrganSrc), _p, C.POINTER(_p)]),
    "hk_organ_free": (C.c_int, [_p, _p]),
    "hk_organ_info": (C.c_int, [_p, C.POINTER(_i32), C.POINTER(_i32), C.POINTER(_u32),
                                C.POINTER(_u32), C.POINTER(_sz)]),
    "hk_gemv": (C.c_int, [_p, _p, _p, _p, _p]),
    "hk_gemv_lowrank": (C.c_int, [_p, _p, _p, _p, _p, _p, _p]),
    "hk_gemv_lowrank_set": (C.c_int, [_p, _p, _p, _p, _sz, _p, _sz, _p, _sz, _p]),
    "hk_organ_upload_rice": (C.c_int, [_p, C.POINTER(RiceQ1Src), _p, C.POINTER(_p)]),
    "hk_rice_apply": (C.c_int, [_p, _p, _p, _p, _p]),
    "hk_terminal_greedy": (C.c_int, [_p, _p, _p, C.c_float, _p, _u32, _p, _p, _p, _p, _p]),
    "hk_terminal_greedy_noalloc": (C.c_int, [_p, _p, _p, C.c_float, _p, _u32, _p, _p]),
    "hk_organ_from_container": (C.c_int, [_p, _i32, _p, _sz, _p, C.POINTER(_p), C.POINTER(_p)]),
    "hk_organ_from_hq30": (C.c_int, [_p, _p, _sz, _p, C.POINTER(_p)]),
    "hk_catalog_open": (C.c_int, [_p, C.c_char_p, C.POINTER(_p)]),
    "hk_catalog_close": (C.c_int, [_p]),
    "hk_catalog_info": (C.c_int, [_p, C.POINTER(_u32), C.POINTER(_u32), C.POINTER(C.c_double), C.POINTER(_u64)]),
    "hk_catalog_record_at": (C.c_int, [_p, _u32, C.POINTER(CatalogRecord)]),
    "hk_catalog_find": (C.c_int, [_p, _p, C.c_char_p, C.POINTER(CatalogRecord)]),
    "hk_catalog_payload": (C.c_int, [_p, _p, C.c_char_p, C.c_int, C.POINTER(_p), C.POINTER(_sz)]),
    "hk_catalog_load": (C.c_int, [_p, _p, C.c_char_p, C.c_int, _p, C.POINTER(_p), C.POINTER(_p)]),
    "hk_pack_binary_rice": (C.c_int, [_p, _p, _u32, _u32, C.c_double, _p, _p, _p, _p, _sz, C.POINTER(RiceQ1Src), _p]),
    "hk_moe_block": (C.c_int, [_p, _p, _u32, _p, _p, _u32, C.c_int, _p, _p, _p]),
    "hk_pack_mixed": (C.c_int, [_p, _p, _u32, _u32, _p, _p, _p, _p, _u32, _p, _p, _u32, C.POINTER(_u32), _p]),
    "hk_organ_from_q4_0": (C.c_int, [_p, _p, _sz, _u32, _u32, _p, C.POINTER(_p)]),
    "hk_gemv_batch": (C.c_int, [_p, C.POINTER(_p), _u32, _p, _sz, _p, _sz, _p]),
    "hk_decode_rows": (C.c_int, [_p, _p, _u32, _u32, _p, _p]),
    "hk_organ_set_create": (C.c_int, [_p, C.POINTER(_p), _u32, C.POINTER(_p)]),
    "hk_organ_set_free": (C.c_int, [_p, _p]),
    "hk_gemv_set": (C.c_int, [_p, _p, _p, _sz, _p, _sz, _p]),
    "hk_organ_synthetic": (C.c_int, [_p, _i32, _i32, _u32, _u32, _u64, _u64, C.c_float, _p, C.POINTER(_p)]),
    "hk_pack_q4": (C.c_int, [_p, _p, _u32, _u32, _i32, _p, _p, _p]),
    "hk_pack_bin": (C.c_int, [_p, _p, _u32, _u32, _p, _p, _p]),
    "hk_pack_q2": (C.c_int, [_p, _p, _sz, _p, _p, _p]),
    "hk_pack_q8": (C.c_int, [_p, _p, _u32, _u32, _p, _p, _p]),
    "hk_pack_u3": (C.c_int, [_p, _p, _sz, _p, _p, _p]),
    "hk_stream_key": (_u64, [_u64, _u64]),
    "hk_synth_normal": (C.c_int, [_p, _u64, _u64, _sz, C.c_float, _p, _p]),
    "hk_router_softmax_topk": (C.c_int, [_p, _p, _u32, _u32, _u32, C.c_float, C.c_int, _p, _p, _p]),
    "hk_router_noaux_tc": (C.c_int, [_p, _p, _p, _u32, _u32, _u32, _u32, _u32, C.c_int, C.c_float,
                                     _p, _p, _p]),
    "hk_moe_model_create": (C.c_int, [_p, C.POINTER(MoeConfig), C.POINTER(_p)]),
    "hk_moe_model_free": (C.c_int, [_p, _p]),
    "hk_moe_model_set_layer": (C.c_int, [_p, _p, _u32, C.POINTER(MoeLayerSrc), _p]),
    "hk_moe_model_fill_synthetic": (C.c_int, [_p, _p, _u64, _p]),
    "hk_moe_stream_id": (_u64, [_u32, _u32, _u32]),
    "hk_moe_model_bytes": (C.c_int, [_p, C.POINTER(_sz), C.POINTER(_sz)]),
    "hk_moe_expert_bytes": (C.c_int, [_p, _u32, _u32, C.POINTER(_sz)]),
    "hk_moe_decode_layer": (C.c_int, [_p, _p, _u32, _p, _p, _p, _p, _p]),
    "hk_moe_decode_stack": (C.c_int, [_p, _p, _p, _p, _p, _p, _p]),
    "hk_moe_decode_stack_persistent": (C.c_int, [_p, _p, _p]),
    "hk_moe_model_set_stack_launch": (C.c_int, [_p, _p, _i32]),
    "hk_moe_model_set_stall_polls": (C.c_int, [_p, _p, _u32]),
    "hk_moe_forward_batch": (C.c_int, [_p, _p, _u32, _p, _u32, _p, _p, _p, _p]),
    "hk_moe15_layer_create": (C.c_int, [_p, C.POINTER(Moe15LayerSrc), C.POINTER(_p)]),
    "hk_moe15_layer_free": (C.c_int, [_p, _p]),
    "hk_moe15_decode_layer": (C.c_int, [_p, _p, _p, _p, _p, _p, _p]),
    "hk_moe15_decode_stack": (C.c_int, [_p, _p, _u32, _p, _p, _p, _p, _p]),
}

_lib: C.CDLL | None = None


class HawkingError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str = ""):
        super().__init__(f"{fn} -> {STATUS_NAMES.get(code, code)}: {msg}")
        self.fn, self.code, self.msg = fn, code, msg


def lib() -> C.CDLL:
    """The loaded library; raises if it is missing (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"HIP library not built: {LIB_PATH} is missing (run `python -m hawking_amd.build`)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols() -> list[str]:
    return list(PROTOTYPES)
