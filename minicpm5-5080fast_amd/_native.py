"""ctypes binding of libminicpm_native.so (the C ABI in include/*.h).

The library is built in-tree by `make -C minicpm5-5080fast_amd/csrc`
(__graft_entry__.build()). There is no fallback: if the library is missing the
import fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libminicpm_native.so")

MC_OK = 0
STATUS_NAMES = {0: "MC_OK", 1: "MC_E_INVALID_ARGUMENT", 2: "MC_E_IO", 3: "MC_E_CUDA",
                4: "MC_E_MODEL_MISMATCH", 5: "MC_E_OUT_OF_MEMORY", 6: "MC_E_GRAPH",
                7: "MC_E_UNSUPPORTED", 100: "MC_E_INTERNAL"}


class McError(RuntimeError):
    def __init__(self, status: int, where: str, message: str):
        super().__init__(f"{where}: {STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class LayoutT(C.Structure):
    _fields_ = [("max_pages", C.c_uint32), ("tokens_per_page", C.c_uint32),
                ("num_layers", C.c_uint32), ("reserved", C.c_uint32)]


_lib = None

_P = C.c_void_p
_u32 = C.c_uint32
_SIGS = {
    # name: (restype, argtypes)
    "mc_last_error": (C.c_char_p, []),
    "mc_kv_build_info": (C.c_char_p, []),
    "mc_kv_elem_offset": (C.c_uint64, [LayoutT] + [_u32] * 6),
    "mc_kv_total_elems": (C.c_uint64, [LayoutT]),
    "mc_kv_decode_chunk_pos": (_u32, [_u32]),
    "mc_kv_decode_max_chunks": (_u32, [_u32, _u32]),
    "mc_kv_prefill_split_kv": (_u32, [_u32]),
    "mc_kv_allocator_create": (C.c_int, [_P, _u32, _u32, C.POINTER(_P)]),
    "mc_kv_allocator_destroy": (None, [_P]),
    "mc_kv_allocator_ensure_pages_for": (C.c_int, [_P, _u32, _P]),
    "mc_kv_allocator_release_all": (None, [_P]),
    "mc_kv_allocator_pages_owned": (_u32, [_P]),
    "mc_kv_allocator_pages_synced": (_u32, [_P]),
    "mc_kv_allocator_host_table": (_u32, [_P, _P, _u32]),
    "mc_kv_pool_create": (C.c_int, [_u32, _u32, _u32, C.POINTER(_P)]),
    "mc_kv_pool_destroy": (None, [_P]),
    "mc_kv_pool_ensure": (C.c_int, [_P, _u32, _u32, _P, _P]),
    "mc_kv_pool_release": (C.c_int, [_P, _u32]),
    "mc_kv_pool_pages_free": (_u32, [_P]),
    "mc_kv_pool_session_pages": (_u32, [_P, _u32]),
    "mc_kv_pool_session_table": (_u32, [_P, _u32, _P, _u32]),
    "mc_kv_rope_inv_freq_init": (C.c_int, [_P, C.c_double, _P]),
    "mc_kv_rope_append": (C.c_int, [_P, _u32, _P, _u32, _P, _P, LayoutT, C.c_double,
                                    _P, _P]),
    "mc_kv_attention_decode": (C.c_int, [_P, _P, _u32, _P, _P, LayoutT, _P, _u32, _P,
                                         _P, _P, _u32, _P]),
    "mc_kv_attention_decode_chunks": (C.c_int, [_P, _P, _u32, _P, _P, LayoutT, _P, _u32,
                                                _P, _P, _P, _u32]),
    "mc_kv_attention_decode_merge": (C.c_int, [_P, _P, _u32, _u32, _P, _P, _P]),
    "mc_kv_attention_decode_batch": (C.c_int, [_P, _P, _u32, _u32, _P, _P, LayoutT, _P,
                                               _u32, _P, _P, _P, _u32, _P]),
    "mc_kv_attention_prefill": (C.c_int, [_P, _u32, _P, _u32, _P, _P, LayoutT, _P, _P,
                                          _u32, _P]),
    "mc_kv_decode_advance": (C.c_int, [_P, _P, _P, _P]),
    "mc_kv_batch_advance": (C.c_int, [_P, _P, _P, _u32, _P]),
    "mc_kv_debug_prefill_shape": (C.c_int, [_u32, _P]),
    "mc_kv_debug_prefill_packing": (C.c_int, [_u32, _P]),
    "mc_kv_debug_prefill_status": (C.c_int, [_P, _u32]),
    "mc_kv_debug_prefill_force_timeouts": (C.c_int, [_u32]),
    "mc_kv_debug_decode_fp32p": (C.c_int, [_u32, _P]),
    "mc_kv_attention_decode_noalloc": (C.c_int, [_P, _P, _u32, _P, _P, LayoutT, _u32, _P, _P,
                                                 _P, _u32]),
    "mc_debug_breakdown_bucket_count": (C.c_int, []),
    "mc_debug_breakdown_bucket_name": (C.c_char_p, [C.c_int]),
    "mc_debug_breakdown_bucket_of": (C.c_int, [C.c_int]),
    "mc_kv_debug_decode_records_only": (C.c_int, [_u32, _P]),
    "mc_kv_debug_decode_timeline": (C.c_int, [_P, _u32]),
    "mc_model_embedding_gather": (C.c_int, [_P, _P, _P, _P, _u32, _u32, _P]),
    "mc_model_rmsnorm_rows": (C.c_int, [_P, _P, _P, _P, _u32, _u32, C.c_float, _P]),
    "mc_model_swiglu_rows": (C.c_int, [_P, _P, _u32, _u32, _P]),
    "mc_model_gemv": (C.c_int, [_P, _P, _u32, _P, _u32, _u32, _u32, _u32, _P]),
    "mc_model_gemm_rows": (C.c_int, [_P, _P, _u32, _P, _u32, _u32, _u32, _u32, _u32, _P]),
    "mc_model_gemv_resnorm": (C.c_int, [_P, _P, _P, _P, _P, _u32, _P, _u32, _u32, _u32,
                                        C.c_float, _P]),
    "mc_model_gemv_swiglu": (C.c_int, [_P, _P, _u32, _P, _u32, _u32, _u32, _u32, _P]),
    "mc_model_gemv_resnorm_swiglu": (C.c_int, [_P, _P, _P, _P, _P, _u32, _P, _u32, _u32, _u32,
                                               C.c_float, _P]),
    "mc_model_argmax_bf16": (C.c_int, [_P, _u32, _u32, _P, _P, _P, _P, _P]),
    "mc_model_wpk_check": (C.c_int, [C.c_char_p, C.POINTER(C.c_uint64)]),
    "mc_model_wpk_fp8_check": (C.c_int, [C.c_char_p, C.POINTER(C.c_uint64)]),
    "mc_model_gemv_fp8": (C.c_int, [_P, _P, _P, _P, _u32, _u32, _P]),
    "mc_model_gemv_fp8_swiglu": (C.c_int, [_P, _P, _P, _P, _u32, _u32, _P]),
    "mc_model_gemv_fp8_resnorm": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _u32, C.c_float, _P]),
    "mc_model_gemv_fp8_resnorm_swiglu": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _u32,
                                                   C.c_float, _P]),
}


def lib():
    """Loads the native library once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(make -C minicpm5-5080fast_amd/csrc); there is no fallback path")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().mc_last_error().decode("utf-8", "replace")


def check(status: int, where: str) -> None:
    if status != MC_OK:
        raise McError(status, where, last_error())


def layout(max_pages: int, tokens_per_page: int, num_layers: int) -> LayoutT:
    return LayoutT(max_pages, tokens_per_page, num_layers, 0)
