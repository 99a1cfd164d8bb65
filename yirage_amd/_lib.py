"""ctypes binding of libyirage_hip.so (declared in include/yirage_hip.h).

The library is built in-tree by yirage_amd.build; nothing here falls back to
another implementation: a missing or stale library raises immediately.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libyirage_hip.so")

YR_OK = 0
DTYPE_F16, DTYPE_BF16, DTYPE_F32, DTYPE_I32, DTYPE_I64 = 940, 941, 950, 955, 965
W_NK, W_KN = 0, 1
(OP_RMSNORM_LINEAR, OP_GATED_MLP, OP_GQA_PREFILL, OP_LINEAR, OP_GQA_DECODE, OP_ATTENTION, OP_MATMUL, OP_UNARY,
 OP_BINARY, OP_REDUCTION, OP_RMSNORM, OP_PACK, OP_COPY_ND, OP_REDUCTION_MAX, OP_EWISE, OP_TB_PROGRAM) = range(1, 17)


class YirageHipError(RuntimeError):
    pass


class PKMeta(ctypes.Structure):
    """yr_pk_meta: device pointers of the reference's meta tensors."""
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "step", "tokens", "input_tokens", "output_tokens", "num_new_tokens", "prompt_lengths",
        "qo_indptr", "paged_kv_indptr", "paged_kv_indices", "paged_kv_last_page_len")]


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("device_id", ctypes.c_int),
        ("num_compute_units", ctypes.c_int),
        ("compute_capability", ctypes.c_int),
        ("wavefront_size", ctypes.c_int),
        ("total_memory", ctypes.c_size_t),
        ("max_shared_memory", ctypes.c_size_t),
        ("clock_khz", ctypes.c_int),
        ("arch_name", ctypes.c_char * 64),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_SZ = ctypes.c_size_t
_F = ctypes.c_float
_U64 = ctypes.c_uint64

# name -> (restype, argtypes); every symbol declared in include/yirage_hip.h
SIGNATURES = {
    "yr_hip_last_error": (ctypes.c_char_p, []),
    "yr_hip_version": (ctypes.c_char_p, []),
    "yr_hip_device_info": (_I, [_I, ctypes.POINTER(DeviceInfo)]),
    "yr_hip_synth_fill": (_I, [_P, _SZ, _I, _U64, _U64, _F, _P]),
    "yr_hip_rmsnorm_linear_workspace": (_SZ, [_I, _I, _I, _I, _I]),
    "yr_hip_gated_mlp_workspace": (_SZ, [_I, _I, _I, _I, _I]),
    "yr_hip_linear_workspace": (_SZ, [_I, _I, _I, _I, _I]),
    "yr_hip_rmsnorm_linear": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _SZ, _P]),
    "yr_hip_gated_mlp": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "yr_hip_linear": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "yr_hip_gqa_decode_workspace": (_SZ, [_I, _I, _I, _I, _I, _I]),
    "yr_hip_gqa_decode_paged": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "yr_hip_gqa_decode_noalloc_max_bytes": (_SZ, []),
    "yr_hip_gqa_decode_paged_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "yr_hip_gqa_prefill": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "yr_hip_argmax": (_I, [_P, _P, _I, _I, _I, _I, _P]),
    "yr_hip_run_fused": (_I, [_I, _I, _P, _I, _P, _I, _P, _P, _SZ, _P]),
    "yr_hip_fused_workspace": (_SZ, [_I, _I, _P]),
    "yr_hip_graph_attention_workspace": (_SZ, [_I, _I, _I, _I, _P]),
    "yr_hip_graph_attention": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _F, _I, _P, _SZ, _P]),
    "yr_hip_graph_pack": (_I, [_P, _P, _I, _I, _I, _I, _P, _I, _P]),
    "yr_hip_graph_copy_nd": (_I, [_P, _P, _I, _P, _P, _P, _I, _P]),
    "yr_hip_graph_reduction_max": (_I, [_P, _P, ctypes.c_int64, _I, ctypes.c_int64, _I, _P]),
    "yr_hip_graph_unary": (_I, [_P, _P, ctypes.c_int64, _I, _F, _F, _I, _P]),
    "yr_hip_graph_ewise": (_I, [_P, _I, _P, _I, _P, _P, _I, _P, _P, _I, _P]),
    "yr_hip_tb_program": (_I, [_P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _P]),
    "yr_hip_tb_program_check": (_I, [_P, _I, _I, _I, _I, _I, _I]),
    "yr_hip_graph_binary": (_I, [_P, _P, _P, _I, _P, _P, _I, _I, _P]),
    "yr_hip_graph_reduction": (_I, [_P, _P, ctypes.c_int64, _I, ctypes.c_int64, _I, _P]),
    "yr_hip_graph_rmsnorm": (_I, [_P, _P, _I, _I, _F, _I, _P]),
    "yr_hip_graph_matmul": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "yr_pk_graph_build": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "yr_pk_graph_free": (None, [_P]),
    "yr_pk_graph_info": (_I, [_P, ctypes.POINTER(ctypes.c_int64), _I]),
    "yr_pk_graph_task": (_I, [_P, _I, ctypes.POINTER(ctypes.c_int64), _I]),
    "yr_pk_graph_simulate": (_I, [_P, _U64, _I, _I, ctypes.c_char_p, _SZ]),
    "yr_pk_graph_export_json": (_I, [_P, ctypes.c_char_p, _SZ, ctypes.POINTER(_SZ)]),
    "yr_pk_create": (_I, [_P, _P, ctypes.POINTER(_P)]),
    "yr_pk_init_batch": (_I, [_P, _P]),
    "yr_pk_launch": (_I, [_P, _P, _I]),
    "yr_pk_iterations": (_I, [_P, ctypes.POINTER(_I)]),
    "yr_pk_set_launch_mode": (_I, [_P, _I]),
    "yr_pk_read_batch": (_I, [_P, ctypes.POINTER(_I), _SZ]),
    "yr_pk_pack_weights": (_I, [_P, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t)]),
    "yr_pk_set_spin_limit": (_I, [_P, ctypes.c_longlong]),
    "yr_pk_status": (_I, [_P, ctypes.POINTER(ctypes.c_int)]),
    "yr_pk_set_profiler": (_I, [_P, _P, _SZ]),
    "yr_pk_reset_status": (_I, [_P]),
    "yr_pk_destroy": (None, [_P]),
    "yr_backend_num_registered": (_I, []),
    "yr_backend_registered_name": (_I, [_I, ctypes.c_char_p, _SZ]),
    "yr_backend_is_available": (_I, [ctypes.c_char_p]),
    "yr_backend_type_from_name": (_I, [ctypes.c_char_p]),
    "yr_backend_default": (_I, [ctypes.c_char_p, _SZ]),
    "yr_backend_compile_flags": (_I, [ctypes.c_char_p, ctypes.c_char_p, _SZ]),
}

_lib = None


def lib():
    """Load the HIP backend library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise YirageHipError(
                f"{LIB_PATH} not found: build it with `python -m yirage_amd.build` "
                "(the hip backend has no fallback path)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().yr_hip_last_error().decode()


def check(rc: int, what: str = "") -> None:
    if rc != YR_OK:
        raise YirageHipError(f"{what or 'yirage_hip'} failed ({rc}): {last_error()}")
