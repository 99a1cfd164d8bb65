"""CPU-side checks of the C ABI: the library loads, exports every symbol that
include/yirage_hip.h declares, and its argument validation / registry paths
work without a GPU (no compute call is made here)."""
import ctypes
import os
import re

import pytest

from yirage_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            src = open(os.path.join(ROOT, "include", fn)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            names.update(re.findall(r"\b(yr_[a-z0-9_]+)\s*\(", src))
    return names


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    declared = _declared_symbols()
    assert len(declared) >= 20
    missing = [n for n in sorted(declared) if not hasattr(L, n)]
    assert not missing, missing
    # the Python binding covers the whole header too
    assert declared <= set(_lib.SIGNATURES), sorted(declared - set(_lib.SIGNATURES))


def test_version_and_error_channel():
    L = _lib.lib()
    assert b"gfx950" in L.yr_hip_version()
    rc = L.yr_hip_rmsnorm_linear(None, None, None, None, 8, 4096, 4096, _lib.DTYPE_F16, _lib.W_KN, 1e-6,
                                 None, 0, None)
    assert rc == -1
    assert "null pointer" in _lib.last_error()
    fake = ctypes.c_void_p(16)
    rc = L.yr_hip_rmsnorm_linear(fake, None, fake, fake, 8, 4095, 4096, _lib.DTYPE_F16, _lib.W_KN, 1e-6,
                                 None, 0, None)
    assert rc == -1 and "multiples of 8" in _lib.last_error()
    rc = L.yr_hip_gated_mlp(fake, fake, fake, fake, 8, 4096, 14336, 123, _lib.W_KN, None, 0, None)
    assert rc == -1 and "dtype" in _lib.last_error()
    # workspace too small is reported, not launched
    need = L.yr_hip_rmsnorm_linear_workspace(8, 4096, 4096, _lib.DTYPE_F16, _lib.W_KN)
    assert need > 0
    rc = L.yr_hip_rmsnorm_linear(fake, None, fake, fake, 8, 4096, 4096, _lib.DTYPE_F16, _lib.W_KN, 1e-6,
                                 fake, need - 1, None)
    assert rc == -3 and "workspace" in _lib.last_error()
    rc = L.yr_hip_gqa_decode_paged(fake, fake, fake, fake, fake, fake, fake, 8, 32, 8, 64, 64, 4096,
                                   _lib.DTYPE_F16, None, 0, None)
    assert rc == -1 and "head_dim" in _lib.last_error()
    rc = L.yr_hip_run_fused(99, 0, None, 0, None, 0, None, None, 0, None)
    assert rc == -1 and "unknown op kind" in _lib.last_error()


def test_workspace_sizes_are_monotone_and_zero_when_unsplit():
    L = _lib.lib()
    assert L.yr_hip_rmsnorm_linear_workspace(8, 512, 4096, _lib.DTYPE_F16, _lib.W_NK) == 0
    assert L.yr_hip_rmsnorm_linear_workspace(8, 512, 4096, _lib.DTYPE_F16, _lib.W_KN) > 0  # stream-K records
    a = L.yr_hip_gated_mlp_workspace(8, 4096, 14336, _lib.DTYPE_BF16, _lib.W_KN)
    b = L.yr_hip_gated_mlp_workspace(8, 8192, 14336, _lib.DTYPE_BF16, _lib.W_KN)
    assert 0 < a <= b
    assert L.yr_hip_gqa_decode_workspace(32, 32, 8, 128, 256, 64) == 0
    assert L.yr_hip_gqa_decode_workspace(8, 32, 8, 128, 4096, 64) > 0


def test_backend_registry_without_gpu():
    L = _lib.lib()
    n = L.yr_backend_num_registered()
    assert n >= 1
    names = []
    for i in range(n):
        buf = ctypes.create_string_buffer(64)
        t = L.yr_backend_registered_name(i, buf, 64)
        names.append((buf.value.decode(), t))
    assert ("hip", 6) in names
    assert L.yr_backend_type_from_name(b"hip") == 6
    assert L.yr_backend_type_from_name(b"cuda") == 0
    assert L.yr_backend_type_from_name(b"nope") == 999
    buf = ctypes.create_string_buffer(256)
    assert L.yr_backend_compile_flags(b"hip", buf, 256) == 0
    assert b"gfx950" in buf.value
    assert L.yr_backend_compile_flags(b"nope", buf, 256) == -1


def test_python_backend_api_lists_hip():
    import yirage_amd as yr

    assert "hip" in yr.get_registered_backends()
    import torch

    if not torch.cuda.is_available():
        assert not yr.is_backend_available("hip")


def test_graph_attention_plan_leaves_decode_beyond_its_tickets():
    """Graph attention with <= 16 query rows runs on the split-KV decode
    kernel only while every group gets an arrival ticket (64 KiB / 4 B =
    16384 groups); beyond that the prefill kernel runs it.  The workspace
    query shows the choice: the decode plan stages an identity page table
    ((3 G + 1) int32, 256-byte aligned) after the 64 KiB ticket region, the
    prefill plan over dense operands needs only the ticket region."""
    L = _lib.lib()
    M, Lk, d = 1, 64, 128

    def ws(G):
        # dense [G][rows][128] operands: Q / O (M rows), K^T given as [G][d][L], V [G][L][d]
        s = (ctypes.c_int64 * 12)(M * 128, 128, 1, Lk * 128, 1, 128, Lk * 128, 128, 1, M * 128, 128, 1)
        return L.yr_hip_graph_attention_workspace(G, M, Lk, d, s)

    tickets = 64 * 1024
    g = 16384
    assert ws(g) == tickets + (((3 * g + 1) * 4 + 255) // 256) * 256
    assert ws(g + 1) == tickets
