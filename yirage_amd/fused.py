"""Torch-tensor front end of the fused HIP operators.

PyTorch supplies device memory and the current stream only; every operator
runs a hand-written gfx950 kernel through the C ABI.  Outputs are allocated
here (the reference allocates them in Python from the generated program's
output directives, python/yirage/kernel.py:393-402), workspaces come from a
per-device cache that is zero-filled once at allocation.
"""
from __future__ import annotations

import ctypes
import struct

import torch

from . import _lib
from ._lib import check, lib

_TORCH_DT = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}
_ws_cache: dict = {}


def dtype_code(t: torch.dtype) -> int:
    try:
        return _TORCH_DT[t]
    except KeyError:
        raise _lib.YirageHipError(f"hip backend: unsupported dtype {t} (float16/bfloat16 only)")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def workspace(nbytes: int, device) -> torch.Tensor | None:
    """Zero-filled scratch shared by the fused operators on one device/stream.
    The kernels return it to all-zero tickets when they finish."""
    if nbytes == 0:
        return None
    key = (torch.device(device).index, torch.cuda.current_stream(device).cuda_stream)
    ws = _ws_cache.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _ws_cache[key] = ws
    return ws


def _check_cuda(*ts):
    for t in ts:
        if t is not None:
            if not t.is_cuda:
                raise _lib.YirageHipError("hip backend: tensors must live on the GPU")
            if not t.is_contiguous():
                raise _lib.YirageHipError("hip backend: tensors must be contiguous (row-major)")


def _same_dtype(x, *others):
    """Every 16-bit operand must share x's dtype (the kernels read them all
    as x's element type)."""
    for t in others:
        if t is not None and t.dtype != x.dtype:
            raise _lib.YirageHipError(f"hip backend: operand dtype {t.dtype} differs from x's {x.dtype}")


def _w_layout_and_n(w: torch.Tensor, k: int, layout: int | None):
    if layout is None:
        layout = _lib.W_KN
    if layout == _lib.W_KN:
        if w.shape[0] != k:
            raise _lib.YirageHipError(f"W shape {tuple(w.shape)} does not match K={k} (KN layout)")
        return layout, w.shape[1]
    if w.shape[1] != k:
        raise _lib.YirageHipError(f"W shape {tuple(w.shape)} does not match K={k} (NK layout)")
    return layout, w.shape[0]


def rmsnorm_linear(x, gamma, w, eps: float = 1e-6, w_layout: int | None = None, out=None):
    """out = (x * rsqrt(mean(x^2) + eps) * gamma) @ W  (fp32 accumulate)."""
    _check_cuda(x, gamma, w)
    _same_dtype(x, gamma, w)
    B, K = x.shape
    layout, N = _w_layout_and_n(w, K, w_layout)
    dt = dtype_code(x.dtype)
    if out is None:
        out = torch.empty((B, N), dtype=x.dtype, device=x.device)
    nb = lib().yr_hip_rmsnorm_linear_workspace(B, K, N, dt, layout)
    ws = workspace(nb, x.device)
    check(lib().yr_hip_rmsnorm_linear(_ptr(x), _ptr(gamma), _ptr(w), _ptr(out), B, K, N, dt, layout, eps,
                                      _ptr(ws), nb, _stream(x.device)), "rmsnorm_linear")
    return out


def gated_mlp(x, w1, w3, w_layout: int | None = None, out=None):
    """out = silu(x @ W1) * (x @ W3)."""
    _check_cuda(x, w1, w3)
    _same_dtype(x, w1, w3)
    B, K = x.shape
    layout, N = _w_layout_and_n(w1, K, w_layout)
    if w3.shape != w1.shape:
        raise _lib.YirageHipError("W1 and W3 shapes differ")
    dt = dtype_code(x.dtype)
    if out is None:
        out = torch.empty((B, N), dtype=x.dtype, device=x.device)
    nb = lib().yr_hip_gated_mlp_workspace(B, K, N, dt, layout)
    ws = workspace(nb, x.device)
    check(lib().yr_hip_gated_mlp(_ptr(x), _ptr(w1), _ptr(w3), _ptr(out), B, K, N, dt, layout,
                                 _ptr(ws), nb, _stream(x.device)), "gated_mlp")
    return out


def linear(x, w, residual=None, w_layout: int | None = _lib.W_NK, out=None):
    """out = x @ W^T (NK layout, torch Linear.weight) or x @ W (KN) (+ residual)."""
    _check_cuda(x, w, residual)
    _same_dtype(x, w, residual)
    B, K = x.shape
    layout, N = _w_layout_and_n(w, K, w_layout)
    dt = dtype_code(x.dtype)
    if out is None:
        out = torch.empty((B, N), dtype=x.dtype, device=x.device)
    nb = lib().yr_hip_linear_workspace(B, K, N, dt, layout)
    ws = workspace(nb, x.device)
    check(lib().yr_hip_linear(_ptr(x), _ptr(w), _ptr(residual), _ptr(out), B, K, N, dt, layout,
                              _ptr(ws), nb, _stream(x.device)), "linear")
    return out


def gqa_decode_paged(q, k_cache, v_cache, kv_indptr, kv_indices, kv_len, max_kv_len: int | None = None, out=None):
    """Paged GQA decode: q[B,Hq,D], caches [P,page,Hkv,D], int32 page table."""
    _check_cuda(q, k_cache, v_cache, kv_indptr, kv_indices, kv_len)
    _same_dtype(q, k_cache, v_cache)
    B, Hq, D = q.shape
    P, page, Hkv, D2 = k_cache.shape
    if D2 != D or v_cache.shape != k_cache.shape:
        raise _lib.YirageHipError("cache shape mismatch")
    for t in (kv_indptr, kv_indices, kv_len):
        if t.dtype != torch.int32:
            raise _lib.YirageHipError("page table tensors must be int32")
    if max_kv_len is None:
        max_kv_len = int(kv_len.max().item())
    dt = dtype_code(q.dtype)
    if out is None:
        out = torch.empty_like(q)
    nb = lib().yr_hip_gqa_decode_workspace(B, Hq, Hkv, D, max_kv_len, page)
    ws = workspace(nb, q.device)
    check(lib().yr_hip_gqa_decode_paged(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(kv_indptr), _ptr(kv_indices),
                                        _ptr(kv_len), _ptr(out), B, Hq, Hkv, D, page, max_kv_len, dt,
                                        _ptr(ws), nb, _stream(q.device)), "gqa_decode_paged")
    return out


def gqa_prefill(q, k, v, causal: bool = True, out=None):
    """Prefill attention q[B,S,Hq,D], k/v[B,S,Hkv,D]."""
    _check_cuda(q, k, v)
    _same_dtype(q, k, v)
    B, S, Hq, D = q.shape
    Hkv = k.shape[2]
    dt = dtype_code(q.dtype)
    if out is None:
        out = torch.empty_like(q)
    check(lib().yr_hip_gqa_prefill(_ptr(q), _ptr(k), _ptr(v), _ptr(out), B, S, Hq, Hkv, D, int(causal), dt,
                                   _stream(q.device)), "gqa_prefill")
    return out


def argmax(x, n_valid: int | None = None, out=None):
    """Row-wise argmax (lowest index on ties) of a 2-D f16/bf16 tensor -> int64."""
    _check_cuda(x)
    rows, n = x.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=x.device)
    check(lib().yr_hip_argmax(_ptr(x), _ptr(out), rows, n, n if n_valid is None else n_valid,
                              dtype_code(x.dtype), _stream(x.device)), "argmax")
    return out


def synth_fill(t: torch.Tensor, seed: int, std: float, offset: int = 0) -> torch.Tensor:
    """Deterministic ~N(0, std) fill on the device (bit-identical to the CPU generator)."""
    _check_cuda(t)
    check(lib().yr_hip_synth_fill(_ptr(t), t.numel(), dtype_code(t.dtype), seed, offset, std,
                                  _stream(t.device)), "synth_fill")
    return t


def float_bits(x: float) -> int:
    return struct.unpack("<i", struct.pack("<f", x))[0]
