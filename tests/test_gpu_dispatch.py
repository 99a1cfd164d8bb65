"""yr_hip_run_fused (the execute_mugraph-shaped launcher,
python/yirage/kernel.py:22-72,411-421) at every BASELINE config: each op
kind, launched through the generic ABI with pointer arrays and an integer
param list, writes bit for bit what the named entry point writes."""
import ctypes
import struct

import pytest
import torch

from yirage_amd import _lib

pytestmark = pytest.mark.gpu


def _randn(shape, std, dtype, gen):
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * std).to(dtype)


def _fused(kind, ins, outs, params):
    L = _lib.lib()
    P = (ctypes.c_int64 * len(params))(*params)
    nb = L.yr_hip_fused_workspace(kind, len(params), P)
    ws = torch.zeros(max(nb, 1), dtype=torch.uint8, device="cuda")
    pi = (ctypes.c_void_p * len(ins))(*[None if t is None else t.data_ptr() for t in ins])
    po = (ctypes.c_void_p * len(outs))(*[t.data_ptr() for t in outs])
    _lib.check(L.yr_hip_run_fused(kind, len(ins), pi, len(outs), po, len(params), P, ctypes.c_void_p(ws.data_ptr()),
                                  nb, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), f"kind {kind}")


def _same(a, b, what):
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{what}: run_fused differs from the named entry"
    print(f"[{what}] bit-identical", flush=True)


def test_run_fused_every_kind_at_baseline_configs():
    import yirage_amd.fused as F

    gen = torch.Generator().manual_seed(0)
    f16, bf16 = _lib.DTYPE_F16, _lib.DTYPE_BF16
    eps_bits = struct.unpack("<i", struct.pack("<f", 1e-6))[0]
    # config 1: RMSNorm + linear, X[8,4096] f16, W[4096,4096] K x N
    print("case run_fused config 1", flush=True)
    x = _randn((8, 4096), 1.0, torch.float16, gen).cuda()
    gamma = torch.ones(4096, dtype=torch.float16, device="cuda")
    w = _randn((4096, 4096), 0.02, torch.float16, gen).cuda()
    out = torch.empty((8, 4096), dtype=torch.float16, device="cuda")
    _fused(_lib.OP_RMSNORM_LINEAR, [x, gamma, w], [out], [8, 4096, 4096, f16, _lib.W_KN, eps_bits])
    _same(out, F.rmsnorm_linear(x, gamma, w, eps=1e-6), "config 1 rmsnorm_linear")
    # linear with residual (N x K weight, the MPK layout)
    r = _randn((8, 4096), 1.0, torch.float16, gen).cuda()
    out = torch.empty_like(r)
    _fused(_lib.OP_LINEAR, [x, w, r], [out], [8, 4096, 4096, f16, _lib.W_NK])
    _same(out, F.linear(x, w, residual=r, w_layout=_lib.W_NK), "linear + residual")
    # config 2a / 2b: gated MLP
    w1 = _randn((4096, 14336), 0.02, torch.bfloat16, gen).cuda()
    w3 = _randn((4096, 14336), 0.02, torch.bfloat16, gen).cuda()
    for B in (8, 128):
        print(f"case run_fused config 2 B={B}", flush=True)
        xb = _randn((B, 4096), 1.0, torch.bfloat16, gen).cuda()
        out = torch.empty((B, 14336), dtype=torch.bfloat16, device="cuda")
        _fused(_lib.OP_GATED_MLP, [xb, w1, w3], [out], [B, 4096, 14336, bf16, _lib.W_KN])
        _same(out, F.gated_mlp(xb, w1, w3), f"config 2 gated_mlp B={B}")
    # config 3: paged GQA decode
    print("case run_fused config 3", flush=True)
    B, Hq, Hkv, L, D, page = 8, 32, 8, 4096, 128, 64
    P = B * L // page
    kc = _randn((P, page, Hkv, D), 1.0, torch.float16, gen).cuda()
    vc = _randn((P, page, Hkv, D), 1.0, torch.float16, gen).cuda()
    indices = torch.randperm(P, generator=gen).to(torch.int32).cuda()
    indptr = (torch.arange(B + 1, dtype=torch.int32) * (L // page)).cuda()
    lens = torch.full((B,), L, dtype=torch.int32).cuda()
    q = _randn((B, Hq, D), 1.0, torch.float16, gen).cuda()
    out = torch.empty_like(q)
    _fused(_lib.OP_GQA_DECODE, [q, kc, vc, indptr, indices, lens], [out], [B, Hq, Hkv, D, page, L, f16])
    _same(out, F.gqa_decode_paged(q, kc, vc, indptr, indices, lens, max_kv_len=L), "config 3 gqa_decode")
    # config 4: causal prefill
    print("case run_fused config 4", flush=True)
    S = 2048
    q = _randn((1, S, 32, D), 1.0, torch.bfloat16, gen).cuda()
    k = _randn((1, S, 8, D), 1.0, torch.bfloat16, gen).cuda()
    v = _randn((1, S, 8, D), 1.0, torch.bfloat16, gen).cuda()
    out = torch.empty_like(q)
    _fused(_lib.OP_GQA_PREFILL, [q, k, v], [out], [1, S, 32, 8, D, 1, bf16])
    _same(out, F.gqa_prefill(q, k, v, causal=True), "config 4 gqa_prefill")
