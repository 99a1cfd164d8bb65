"""GPU parity of the fused operators against the CPU oracle.

Inputs are drawn on the CPU with torch.Generator seed 0 and copied to the
device, so both sides see identical bits.
Tolerance for 16-bit outputs: rtol 1e-2 / atol 1e-2 against the
double-accumulated oracle; argmax is bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-2
DT = {torch.float16: "f16", torch.bfloat16: "bf16"}


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _f(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def _randn(shape, std, dtype, gen):
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * std).to(dtype)


def _close(got: torch.Tensor, ref: np.ndarray, what: str):
    g = _f(got)
    err = np.abs(g - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    print(f"[{what}] max abs err {err.max():.3e}, mismatches {bad.sum()}/{bad.size}", flush=True)
    assert not bad.any(), f"{what}: {bad.sum()} elements outside rtol/atol 1e-2"


@pytest.mark.parametrize("B,K,N,layout", [(8, 4096, 4096, 1), (3, 1024, 776, 1), (1, 4096, 4096, 0),
                                          (8, 4096, 6144, 0), (5, 14336, 4096, 0), (20, 512, 256, 1),
                                          (37, 1024, 200, 1), (128, 4096, 4096, 1), (128, 4096, 4096, 0),
                                          (45, 1000, 264, 0)])
def test_rmsnorm_linear(B, K, N, layout):
    import yirage_amd.fused as F

    print(f"case rmsnorm_linear B={B} K={K} N={N} layout={layout}", flush=True)
    g = torch.Generator().manual_seed(0)
    x = _randn((B, K), 1.0, torch.float16, g)
    gamma = (1.0 + 0.1 * torch.randn(K, generator=g)).to(torch.float16)
    wshape = (K, N) if layout == 1 else (N, K)
    w = _randn(wshape, 0.02, torch.float16, g)
    out = F.rmsnorm_linear(x.cuda(), gamma.cuda(), w.cuda(), eps=1e-6, w_layout=layout)
    torch.cuda.synchronize()
    ref = O.rmsnorm_linear(_f(x), _f(gamma), _bits(w), "f16", layout, 1e-6)
    _close(out, ref, "rmsnorm_linear")
    # second call reuses the workspace (tickets must have been re-armed)
    out2 = F.rmsnorm_linear(x.cuda(), gamma.cuda(), w.cuda(), eps=1e-6, w_layout=layout)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "non-deterministic result across calls"


def test_rmsnorm_linear_config1_gamma_one():
    """BASELINE config 1 exactly: X[8,4096] f16 ~N(0,1), gamma = 1, W[4096,4096] ~N(0,0.02)."""
    import yirage_amd.fused as F

    g = torch.Generator().manual_seed(0)
    x = _randn((8, 4096), 1.0, torch.float16, g)
    w = _randn((4096, 4096), 0.02, torch.float16, g)
    gamma = torch.ones(4096, dtype=torch.float16)
    out = F.rmsnorm_linear(x.cuda(), gamma.cuda(), w.cuda(), eps=1e-6)
    torch.cuda.synchronize()
    _close(out, O.rmsnorm_linear(_f(x), _f(gamma), _bits(w), "f16", 1, 1e-6), "config1")


@pytest.mark.parametrize("B,K,N,layout", [(8, 4096, 14336, 1), (2, 2048, 520, 1), (8, 4096, 2048, 0),
                                          (1, 4096, 14336, 0), (130, 1024, 520, 1), (140, 1024, 520, 0),
                                          (128, 4096, 14336, 0)])
def test_gated_mlp(B, K, N, layout):
    import yirage_amd.fused as F

    print(f"case gated_mlp B={B} K={K} N={N} layout={layout}", flush=True)
    g = torch.Generator().manual_seed(0)
    x = _randn((B, K), 1.0, torch.bfloat16, g)
    wshape = (K, N) if layout == 1 else (N, K)
    w1 = _randn(wshape, 0.02, torch.bfloat16, g)
    w3 = _randn(wshape, 0.02, torch.bfloat16, g)
    out = F.gated_mlp(x.cuda(), w1.cuda(), w3.cuda(), w_layout=layout)
    torch.cuda.synchronize()
    O.set_num_threads(16)
    ref = O.gated_mlp(_f(x), _bits(w1), _bits(w3), "bf16", layout)
    _close(out, ref, "gated_mlp")


def test_gated_mlp_batch128_all_columns():
    """Config 2b (batch 128, the MFMA path): every one of the 14336 columns
    against the oracle."""
    import yirage_amd.fused as F

    g = torch.Generator().manual_seed(0)
    B, K, N = 128, 4096, 14336
    x = _randn((B, K), 1.0, torch.bfloat16, g)
    w1 = _randn((K, N), 0.02, torch.bfloat16, g)
    w3 = _randn((K, N), 0.02, torch.bfloat16, g)
    out = F.gated_mlp(x.cuda(), w1.cuda(), w3.cuda())
    torch.cuda.synchronize()
    O.set_num_threads(16)
    ref = O.gated_mlp(_f(x), _bits(w1), _bits(w3), "bf16", 1)
    _close(out, ref, "gated_mlp_b128")


@pytest.mark.parametrize("B,K,N,layout,kind", [(17, 1000, 12296, 1, "linear"), (100, 1000, 12296, 0, "linear"),
                                               (33, 1000, 12296, 0, "gated"), (64, 2048, 12296, 1, "rmsnorm"),
                                               (128, 1000, 12296, 0, "rmsnorm")])
def test_batch128_wide_tiles_and_edges(B, K, N, layout, kind):
    """Batches of 17..128 rows with N >= 12288: the direct-to-LDS kernel's
    128-column tiles with two K splits (linear, N x K gated), the last tile 8
    columns wide (N = 96 * 128 + 8) and a partial 64-row chunk in each split
    (K = 1000: splits of 512 and 488 rows); RMSNorm runs in the
    register-staged kernel."""
    import yirage_amd.fused as F

    print(f"case batch128 {kind} B={B} K={K} N={N} layout={layout}", flush=True)
    g = torch.Generator().manual_seed(1)
    x = _randn((B, K), 1.0, torch.bfloat16, g)
    wshape = (K, N) if layout == 1 else (N, K)
    w = _randn(wshape, 0.02, torch.bfloat16, g)
    lay = O.W_KN if layout == 1 else O.W_NK
    O.set_num_threads(16)
    if kind == "linear":
        out = F.linear(x.cuda(), w.cuda(), w_layout=layout)
        ref = O.linear(_f(x), _bits(w), "bf16", lay, None)
    elif kind == "gated":
        w3 = _randn(wshape, 0.02, torch.bfloat16, g)
        out = F.gated_mlp(x.cuda(), w.cuda(), w3.cuda(), w_layout=layout)
        ref = O.gated_mlp(_f(x), _bits(w), _bits(w3), "bf16", layout)
    else:
        gamma = (1.0 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
        out = F.rmsnorm_linear(x.cuda(), gamma.cuda(), w.cuda(), eps=1e-6, w_layout=layout)
        ref = O.rmsnorm_linear(_f(x), _f(gamma), _bits(w), "bf16", layout, 1e-6)
    torch.cuda.synchronize()
    _close(out, ref, f"batch128 {kind}")


@pytest.mark.parametrize("dtype,layout,B", [(torch.float16, 0, 4), (torch.bfloat16, 0, 4), (torch.bfloat16, 1, 4),
                                            (torch.float16, 1, 4), (torch.bfloat16, 1, 40), (torch.bfloat16, 0, 64),
                                            (torch.float16, 0, 150), (torch.bfloat16, 0, 256)])
def test_linear_with_residual(dtype, layout, B):
    import yirage_amd.fused as F

    print(f"case linear+residual {dtype} layout={layout} B={B}", flush=True)
    g = torch.Generator().manual_seed(0)
    K, N = 4096, 1040
    x = _randn((B, K), 1.0, dtype, g)
    w = _randn((N, K) if layout == 0 else (K, N), 0.02, dtype, g)
    r = _randn((B, N), 1.0, dtype, g)
    out = F.linear(x.cuda(), w.cuda(), residual=r.cuda(), w_layout=layout)
    torch.cuda.synchronize()
    ref = O.linear(_f(x), _bits(w), DT[dtype], O.W_NK if layout == 0 else O.W_KN, _f(r))
    _close(out, ref, "linear+residual")


def _paged_cache(B, L, Hkv, D, page, dtype, gen, pool_extra=0):
    npg = (L + page - 1) // page
    P = B * npg + pool_extra
    kc = _randn((P, page, Hkv, D), 1.0, dtype, gen)
    vc = _randn((P, page, Hkv, D), 1.0, dtype, gen)
    perm = torch.randperm(P, generator=gen).to(torch.int32)
    indptr = torch.arange(0, B + 1, dtype=torch.int32) * npg
    return kc, vc, perm[: B * npg].contiguous(), indptr


@pytest.mark.parametrize("B,Hq,Hkv,L,page,dtype", [
    (8, 32, 8, 4096, 64, torch.float16),
    (2, 32, 8, 1000, 64, torch.bfloat16),    # ragged tail
    (3, 8, 8, 300, 16, torch.float16),       # MHA, small pages
    (1, 16, 2, 64, 64, torch.bfloat16),      # single split
    (2, 32, 2, 2000, 1, torch.bfloat16),     # G = 16, one token per page
    (1, 64, 8, 777, 32, torch.float16),      # G = 8
    (40, 32, 8, 200, 16, torch.float16),     # batch * kv heads >= CUs: one split each
])
def test_gqa_decode_paged(B, Hq, Hkv, L, page, dtype):
    import yirage_amd.fused as F

    print(f"case gqa_decode B={B} Hq={Hq} Hkv={Hkv} L={L} page={page} {dtype}", flush=True)
    g = torch.Generator().manual_seed(0)
    D = 128
    kc, vc, indices, indptr = _paged_cache(B, L, Hkv, D, page, dtype, g, pool_extra=3)
    q = _randn((B, Hq, D), 1.0, dtype, g)
    lens = torch.full((B,), L, dtype=torch.int32)
    if B > 1:
        lens[-1] = max(1, L - 37)  # ragged lengths inside one batch
    args = (q.cuda(), kc.cuda(), vc.cuda(), indptr.cuda(), indices.cuda(), lens.cuda())
    out = F.gqa_decode_paged(*args, max_kv_len=L)
    again = F.gqa_decode_paged(*args, max_kv_len=L)  # tickets re-armed: same bits
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    ref = O.gqa_decode_paged(_f(q), _bits(kc), _bits(vc), DT[dtype], indptr.numpy(), indices.numpy(), lens.numpy())
    _close(out, ref, "gqa_decode")


@pytest.mark.parametrize("S,causal,dtype,B,Hq,Hkv", [
    (2048, True, torch.bfloat16, 1, 32, 8),
    (300, True, torch.float16, 1, 32, 8),    # odd block count: the middle block runs alone
    (200, False, torch.bfloat16, 1, 32, 8),
    (300, True, torch.float16, 1, 8, 8),     # MHA (one head per wave)
    (130, True, torch.bfloat16, 2, 6, 2),    # odd group size, batch 2
    (77, False, torch.float16, 2, 4, 1),
    (64, False, torch.bfloat16, 1, 4, 1),    # one full tile, no masked positions
    (1, True, torch.float16, 1, 4, 2),       # single token: output is V
    # more group sizes and ragged lengths: odd block counts, partial last
    # blocks and tiles, a single block, group size 8
    (97, True, torch.bfloat16, 1, 8, 2),
    (33, True, torch.float16, 2, 4, 1),
    (32, True, torch.bfloat16, 1, 4, 1),
    (160, False, torch.bfloat16, 1, 16, 2),  # group size 8, odd block count, one block split
    (1000, True, torch.float16, 1, 8, 1),    # group size 8, causal
])
def test_gqa_prefill(S, causal, dtype, B, Hq, Hkv):
    import yirage_amd.fused as F

    print(f"case gqa_prefill S={S} causal={causal} {dtype} B={B} Hq={Hq} Hkv={Hkv}", flush=True)
    g = torch.Generator().manual_seed(0)
    D = 128
    q = _randn((B, S, Hq, D), 1.0, dtype, g)
    k = _randn((B, S, Hkv, D), 1.0, dtype, g)
    v = _randn((B, S, Hkv, D), 1.0, dtype, g)
    out = F.gqa_prefill(q.cuda(), k.cuda(), v.cuda(), causal=causal)
    torch.cuda.synchronize()
    # every query row of every head against the oracle
    O.set_num_threads(16)
    ref = O.gqa_prefill(_f(q), _f(k), _f(v), causal=causal)
    _close(out, ref, "gqa_prefill")


def test_argmax_planted_and_ties():
    """Known answer of tests/runtime_python/test_argmax.py:9-34 plus ties."""
    import yirage_amd.fused as F

    g = torch.Generator().manual_seed(0)
    rows, V = 6, 153600
    x = torch.randn((rows, V), generator=g).to(torch.bfloat16)
    idx = torch.randint(0, V, (rows,), generator=g)
    x[torch.arange(rows), idx] = 65504.0
    x[1, 5] = 65504.0  # tie at a lower index than the planted one (unless planted < 5)
    got = F.argmax(x.cuda())
    torch.cuda.synchronize()
    ref = O.argmax(_f(x))
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
    # padding mask: n_valid excludes the tail
    y = torch.full((2, 1000), -3.0, dtype=torch.bfloat16)
    y[:, 990:] = 0.0
    y[0, 7] = -1.0
    np.testing.assert_array_equal(F.argmax(y.cuda(), n_valid=990).cpu().numpy(), [7, 0])


def test_synth_fill_bit_identical_to_cpu():
    import yirage_amd.fused as F

    for dt, name in ((torch.bfloat16, "bf16"), (torch.float16, "f16")):
        t = torch.empty(1 << 20, dtype=dt, device="cuda")
        F.synth_fill(t, seed=1234, std=0.02, offset=77)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(t), O.synth((1 << 20,), name, seed=1234, std=0.02, offset=77))
