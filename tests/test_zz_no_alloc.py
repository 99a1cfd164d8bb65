"""GPU check of yr_hip_gqa_decode_paged_noalloc, the decode entry point that
allocates nothing (its tickets and split records live in a fixed device
array): called through the C ABI, its output must equal, bit for bit, what
yr_hip_gqa_decode_paged writes for the same inputs, on two calls in a row,
the second one smaller (the array keeps the first call's contents)."""
import ctypes

import pytest
import torch

from yirage_amd import _lib

pytestmark = pytest.mark.gpu


def _case(B, Hq, Hkv, L, page, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    D = 128
    npg = (L + page - 1) // page
    P = B * npg + 3
    kc = torch.randn((P, page, Hkv, D), generator=g).to(dtype).cuda()
    vc = torch.randn((P, page, Hkv, D), generator=g).to(dtype).cuda()
    indices = torch.randperm(P, generator=g)[: B * npg].to(torch.int32).cuda()
    indptr = (torch.arange(B + 1, dtype=torch.int32) * npg).cuda()
    lens = torch.full((B,), L, dtype=torch.int32)
    if B > 1:
        lens[-1] = max(1, L - 37)
    q = torch.randn((B, Hq, D), generator=g).to(dtype).cuda()
    return q, kc, vc, indptr, indices, lens.cuda()


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def test_noalloc_decode_matches_workspace_entry():
    L_ = _lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dt_code = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}
    cases = [(8, 32, 8, 4096, 64, torch.float16, 0),
             (2, 32, 8, 1000, 64, torch.bfloat16, 1)]  # second call, smaller
    for B, Hq, Hkv, L, page, dtype, seed in cases:
        print(f"case noalloc decode B={B} Hq={Hq} Hkv={Hkv} L={L} page={page} {dtype}", flush=True)
        q, kc, vc, indptr, indices, lens = _case(B, Hq, Hkv, L, page, dtype, seed)
        D, dt = 128, dt_code[dtype]
        need = L_.yr_hip_gqa_decode_workspace(B, Hq, Hkv, D, L, page)
        assert 0 < need <= L_.yr_hip_gqa_decode_noalloc_max_bytes()
        ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
        ref = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        _lib.check(L_.yr_hip_gqa_decode_paged(_p(q), _p(kc), _p(vc), _p(indptr), _p(indices), _p(lens), _p(ref),
                                              B, Hq, Hkv, D, page, L, dt, _p(ws), need, stream), "decode")
        _lib.check(L_.yr_hip_gqa_decode_paged_noalloc(_p(q), _p(kc), _p(vc), _p(indptr), _p(indices), _p(lens),
                                                      _p(got), B, Hq, Hkv, D, page, L, dt, stream), "noalloc")
        torch.cuda.synchronize()
        assert torch.equal(ref.view(torch.int16), got.view(torch.int16)), "noalloc output differs"
