"""ctypes/numpy front end of the CPU oracle (oracle/yr_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker.  The yirage_amd product
path never imports this module.

Every function takes/returns numpy arrays.  16-bit tensors travel as uint16
storage with a dtype tag ("f16" or "bf16"); activations are float32 arrays
whose values are representable in the tagged dtype when the reference keeps
them in that dtype.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

F16, BF16 = 0, 1
W_NK, W_KN = 0, 1
_DT = {"f16": F16, "fp16": F16, "float16": F16, "bf16": BF16, "bfloat16": BF16}


def build(force: bool = False) -> str:
    src = os.path.join(_HERE, "yr_oracle.c")
    if force or not os.path.exists(_LIB_PATH) or os.path.getmtime(_LIB_PATH) < os.path.getmtime(src):
        subprocess.check_call(["make", "-s", "-C", _HERE, "liboracle.so"])
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i32, i64, u64, f32, sz = ctypes.c_int, ctypes.c_longlong, ctypes.c_uint64, ctypes.c_float, ctypes.c_size_t
        sig = {
            "yo_to_float": (None, [P, sz, i32, P]),
            "yo_from_float": (None, [P, sz, i32, P]),
            "yo_round": (None, [P, sz, i32]),
            "yo_synth_fill": (None, [P, sz, i32, u64, u64, f32]),
            "yo_synth_fill_float": (None, [P, sz, i32, u64, u64, f32]),
            "yo_synth_scale": (f32, [f32]),
            "yo_rmsnorm": (None, [P, i32, i32, P, f32, P]),
            "yo_linear": (None, [P, i32, i32, P, i32, i32, i32, P, P]),
            "yo_rmsnorm_linear": (None, [P, i32, i32, P, f32, P, i32, i32, i32, P]),
            "yo_gated_mlp": (None, [P, i32, i32, P, P, i32, i32, i32, P]),
            "yo_silu_mul": (None, [P, P, sz, i32, P]),
            "yo_rope": (None, [P, i32, i32, P, P, i32]),
            "yo_gqa_decode_paged": (None, [P, i32, i32, i32, i32, P, P, i32, i32, P, P, P, P]),
            "yo_gqa_prefill": (None, [P, P, P, i32, i32, i32, i32, i32, i32, P, i32, P]),
            "yo_paged_attention": (None, [P, i32, i32, i32, P, P, i32, i32, i32, P, P, P, P, P, P, P, P, f32,
                                          P]),
            "yo_argmax": (None, [P, i32, i32, i32, P]),
            "yo_batch_init": (None, [P]),
            "yo_batch_prepare_next": (i32, [P]),
            "yo_batch_prepare_online": (i32, [P, P]),
            "yo_num_threads": (i32, []),
            "yo_set_num_threads": (None, [i32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def dt_code(dt) -> int:
    return _DT[dt] if isinstance(dt, str) else int(dt)


# ---------------------------------------------------------------- conversions

def to_float(bits: np.ndarray, dt) -> np.ndarray:
    bits = _c(bits, np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().yo_to_float(_p(bits), bits.size, dt_code(dt), _p(out))
    return out


def from_float(x: np.ndarray, dt) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().yo_from_float(_p(x), x.size, dt_code(dt), _p(out))
    return out


def round_to(x: np.ndarray, dt) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    lib().yo_round(_p(y), y.size, dt_code(dt))
    return y


def synth(shape, dt, seed: int, std: float, offset: int = 0) -> np.ndarray:
    """Deterministic ~N(0, std) tensor as uint16 storage (same bits as the
    device generator yr_hip_synth_fill)."""
    out = np.empty(shape, np.uint16)
    lib().yo_synth_fill(_p(out), out.size, dt_code(dt), ctypes.c_uint64(seed), ctypes.c_uint64(offset), std)
    return out


def synth_float(shape, dt, seed: int, std: float, offset: int = 0) -> np.ndarray:
    out = np.empty(shape, np.float32)
    lib().yo_synth_fill_float(_p(out), out.size, dt_code(dt), ctypes.c_uint64(seed), ctypes.c_uint64(offset), std)
    return out


# ---------------------------------------------------------------- operators

def rmsnorm(x: np.ndarray, w: np.ndarray | None, eps: float = 1e-6) -> np.ndarray:
    x = _c(x, np.float32)
    rows, H = x.reshape(-1, x.shape[-1]).shape
    out = np.empty_like(x)
    wf = None if w is None else _c(w, np.float32)
    lib().yo_rmsnorm(_p(x), rows, H, _p(wf), eps, _p(out))
    return out


def linear(x: np.ndarray, W: np.ndarray, wdt, layout: int, residual: np.ndarray | None = None) -> np.ndarray:
    x = _c(x, np.float32)
    W = _c(W, np.uint16)
    B, K = x.shape
    N = W.shape[0] if layout == W_NK else W.shape[1]
    assert (W.shape == (N, K)) if layout == W_NK else (W.shape == (K, N))
    out = np.empty((B, N), np.float32)
    r = None if residual is None else _c(residual, np.float32)
    lib().yo_linear(_p(x), B, K, _p(W), dt_code(wdt), layout, N, _p(r), _p(out))
    return out


def rmsnorm_linear(x, gamma, W, wdt, layout=W_KN, eps=1e-6):
    x = _c(x, np.float32)
    g = None if gamma is None else _c(gamma, np.float32)
    W = _c(W, np.uint16)
    B, K = x.shape
    N = W.shape[1] if layout == W_KN else W.shape[0]
    out = np.empty((B, N), np.float32)
    lib().yo_rmsnorm_linear(_p(x), B, K, _p(g), eps, _p(W), dt_code(wdt), layout, N, _p(out))
    return out


def gated_mlp(x, W1, W3, wdt, layout=W_KN):
    x = _c(x, np.float32)
    W1 = _c(W1, np.uint16)
    W3 = _c(W3, np.uint16)
    B, K = x.shape
    N = W1.shape[1] if layout == W_KN else W1.shape[0]
    out = np.empty((B, N), np.float32)
    lib().yo_gated_mlp(_p(x), B, K, _p(W1), _p(W3), dt_code(wdt), layout, N, _p(out))
    return out


def silu_mul(gate, up, dt):
    g = _c(gate, np.float32)
    u = _c(up, np.float32)
    out = np.empty_like(g)
    lib().yo_silu_mul(_p(g), _p(u), g.size, dt_code(dt), _p(out))
    return out


def rope(x, cos_row, sin_row, dt):
    """x: [n_heads, D] float (rotated copy returned)."""
    y = np.array(x, np.float32, copy=True, order="C")
    nh, D = y.shape
    lib().yo_rope(_p(y), nh, D, _p(_c(cos_row, np.float32)), _p(_c(sin_row, np.float32)), dt_code(dt))
    return y


def gqa_decode_paged(q, kc, vc, dt, kv_indptr, kv_indices, kv_len):
    """q [B,Hq,D] float; kc/vc [P,page,Hkv,D] uint16."""
    q = _c(q, np.float32)
    kc = _c(kc, np.uint16)
    vc = _c(vc, np.uint16)
    B, Hq, D = q.shape
    _, page, Hkv, D2 = kc.shape
    assert D2 == D
    out = np.empty_like(q)
    lib().yo_gqa_decode_paged(_p(q), B, Hq, Hkv, D, _p(kc), _p(vc), dt_code(dt), page,
                              _p(_c(kv_indptr, np.int32)), _p(_c(kv_indices, np.int32)),
                              _p(_c(kv_len, np.int32)), _p(out))
    return out


def gqa_prefill(q, k, v, causal=True, rows=None):
    """q [B,S,Hq,D], k/v [B,S,Hkv,D] float.  rows: optional subset of query rows."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    B, S, Hq, D = q.shape
    Hkv = k.shape[2]
    out = np.zeros_like(q)
    if rows is None:
        lib().yo_gqa_prefill(_p(q), _p(k), _p(v), B, S, Hq, Hkv, D, int(causal), None, -1, _p(out))
    else:
        r = _c(rows, np.int32)
        lib().yo_gqa_prefill(_p(q), _p(k), _p(v), B, S, Hq, Hkv, D, int(causal), _p(r), r.size, _p(out))
    return out


def paged_attention(qkv, Hq, Hkv, D, kc, vc, dt, qo_indptr, kv_indptr, kv_indices, last_page_len,
                    cos_t=None, sin_t=None, q_norm=None, k_norm=None, qk_eps=1e-6):
    """MPK attention task; kc/vc are updated in place (new tokens appended).
    q_norm / k_norm: per-head RMSNorm weights [D] applied before RoPE."""
    qkv = _c(qkv, np.float32)
    assert kc.dtype == np.uint16 and kc.flags.c_contiguous and vc.flags.c_contiguous
    page = kc.shape[1]
    R = len(qo_indptr) - 1
    T = qkv.shape[0]
    out = np.zeros((T, Hq * D), np.float32)
    ct = None if cos_t is None else _c(cos_t, np.float32)
    st = None if sin_t is None else _c(sin_t, np.float32)
    lib().yo_paged_attention(_p(qkv), Hq, Hkv, D, _p(kc), _p(vc), dt_code(dt), page, R,
                             _p(_c(qo_indptr, np.int32)), _p(_c(kv_indptr, np.int32)),
                             _p(_c(kv_indices, np.int32)), _p(_c(last_page_len, np.int32)),
                             _p(ct), _p(st), _p(None if q_norm is None else _c(q_norm, np.float32)),
                             _p(None if k_norm is None else _c(k_norm, np.float32)), float(qk_eps), _p(out))
    return out


def argmax(x, n_valid=None):
    x = _c(x, np.float32)
    rows, V = x.shape
    out = np.empty(rows, np.int64)
    lib().yo_argmax(_p(x), rows, V, V if n_valid is None else int(n_valid), _p(out))
    return out


# ---------------------------------------------------------------- page manager

class _BatchState(ctypes.Structure):
    _fields_ = [
        ("max_requests", ctypes.c_int), ("max_tokens", ctypes.c_int), ("max_pages", ctypes.c_int),
        ("page_size", ctypes.c_int), ("max_seq_length", ctypes.c_int),
        ("total_num_requests", ctypes.c_int), ("eos_token_id", ctypes.c_longlong),
    ] + [(n, ctypes.c_void_p) for n in (
        "step", "tokens", "input_tokens", "output_tokens", "prompt_length", "qo_indptr", "kv_indptr",
        "kv_indices", "last_page_len", "request_ids", "next_request_id", "page_queue",
        "page_queue_head", "page_queue_tail")]


class BatchManager:
    """Offline batch/page manager (persistent_kernel.cuh:107-132,169-322) over
    numpy arrays that mirror the reference meta tensors."""

    def __init__(self, max_requests, max_tokens, max_pages, page_size, tokens, prompt_lengths, eos):
        self.a = {
            "step": np.zeros(tokens.shape[0], np.int32),
            "tokens": np.ascontiguousarray(tokens, np.int64),
            "input_tokens": np.zeros(max_tokens, np.int64),
            "output_tokens": np.zeros(max_tokens, np.int64),
            "prompt_length": np.ascontiguousarray(prompt_lengths, np.int32),
            "qo_indptr": np.zeros(max_requests + 1, np.int32),
            "kv_indptr": np.zeros(max_requests + 1, np.int32),
            "kv_indices": np.zeros(max_pages, np.int32),
            "last_page_len": np.zeros(max_requests, np.int32),
            "request_ids": np.zeros(max_requests, np.int32),
            "next_request_id": np.zeros(1, np.int32),
            "page_queue": np.zeros(max_pages, np.int32),
            "page_queue_head": np.zeros(1, np.int32),
            "page_queue_tail": np.zeros(1, np.int32),
        }
        s = _BatchState()
        s.max_requests, s.max_tokens, s.max_pages = max_requests, max_tokens, max_pages
        s.page_size, s.max_seq_length = page_size, tokens.shape[1]
        s.total_num_requests, s.eos_token_id = tokens.shape[0], eos
        for k, v in self.a.items():
            setattr(s, k, v.ctypes.data)
        self.s = s
        lib().yo_batch_init(ctypes.byref(s))

    def prepare_next(self) -> bool:
        return bool(lib().yo_batch_prepare_next(ctypes.byref(self.s)))

    def prepare_online(self, new_token_nums) -> bool:
        """Online mode (persistent_kernel.cuh:325-351): step[0] advances by
        new_token_nums[0]; False once the sequence ends."""
        n = np.ascontiguousarray(new_token_nums, np.int32)
        return bool(lib().yo_batch_prepare_online(ctypes.byref(self.s), _p(n)))

    def __getitem__(self, k):
        return self.a[k]


def set_num_threads(n: int):
    lib().yo_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().yo_num_threads())
