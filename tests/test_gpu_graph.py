"""GPU parity of the kernel-graph front end: graphs built as the reference's
benchmarks, demos and tests build them (benchmark/{rmsnorm,gated_mlp,
group_query_attention}.py, demo/reference_mugraphs/*.py,
tests/python/test_tensor_program.py), superoptimized for the `hip` backend
and called.

  * fused patterns: bit-identical to the direct fused entry points (same
    kernels) and within rtol/atol 1e-2 of the CPU oracle at BASELINE configs
    1, 2a, 2b; the attention pattern against the decode (config 3 shape) and
    prefill (config 4 shape, non-causal: the graph vocabulary has no mask)
    kernels, with the graph's unscaled softmax checked against the oracle;
  * generic ops (graphs no pattern covers): within 1e-2 of a torch float64
    reference that rounds to 16 bits after every op, as the kernels do.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

import yirage_amd as yr
from oracle import oracle as O
from yirage_amd import _lib

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-2


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _f(t):
    return t.detach().float().cpu().numpy()


def _randn(shape, std, dtype, gen):
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * std).to(dtype)


def _close(got, ref, what, rtol=RTOL, atol=ATOL):
    g = _f(got) if isinstance(got, torch.Tensor) else got
    err = np.abs(g - ref)
    bad = err > atol + rtol * np.abs(ref)
    print(f"[{what}] max abs err {err.max():.3e}, mismatches {bad.sum()}/{bad.size}", flush=True)
    assert not bad.any(), f"{what}: {bad.sum()} elements outside rtol/atol"


def _same_bits(a, b, what):
    assert torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16)), f"{what}: bits differ"


def test_graph_rmsnorm_linear_config1():
    import yirage_amd.fused as F

    print("case graph rms_norm + matmul, config 1", flush=True)
    g = torch.Generator().manual_seed(0)
    x = _randn((8, 4096), 1.0, torch.float16, g)
    w = _randn((4096, 4096), 0.02, torch.float16, g)
    graph = yr.new_kernel_graph()
    X = graph.new_input(dims=(8, 4096), dtype=yr.float16)
    W = graph.new_input(dims=(4096, 4096), dtype=yr.float16)
    graph.mark_output(graph.matmul(graph.rms_norm(X, normalized_shape=(4096,)), W))
    opt = graph.superoptimize(backend="hip", warmup_iters=2, profile_iters=5, use_graph_dataset=False)
    assert opt.backend == "hip" and opt._plan.describe() == ["rmsnorm_linear"], opt._plan.describe()
    out = opt(inputs=[x.cuda(), w.cuda()])[0]
    direct = F.rmsnorm_linear(x.cuda(), torch.ones(4096, dtype=torch.float16, device="cuda"), w.cuda(), eps=1e-6)
    torch.cuda.synchronize()
    _same_bits(out, direct, "graph vs direct rmsnorm_linear")
    _close(out, O.rmsnorm_linear(_f(x), None, _bits(w), "f16", 1, 1e-6), "graph config1")


def test_graph_rmsnorm_linear_customized_column_major():
    """tests/python/test_tensor_program.py:380-435: the customized RMSNorm
    threadblock graph over column-major X (8 x 4096, strides (1, 8)) and W
    (strides (1, 4096), i.e. W stored N x K)."""
    print("case customized rms_norm, column-major inputs", flush=True)
    g = torch.Generator().manual_seed(1)
    xs = (torch.rand((4096, 8), generator=g) * -0.5 + 1).half()      # storage of X^T
    ws = (torch.rand((4096, 4096), generator=g) * -0.5 + 1).half()   # storage of W^T
    graph = yr.new_kernel_graph()
    X = graph.new_input((8, 4096), (1, 8), dtype=yr.float16)
    W = graph.new_input((4096, 4096), (1, 4096), dtype=yr.float16)
    tb = yr.new_threadblock_graph(grid_dim=(64, 1, 1), block_dim=(128, 1, 1), forloop_range=64, reduction_dimx=64)
    tX = tb.new_input(dtensor=X, input_map=(-1, -1, -1), forloop_dim=1)
    tW = tb.new_input(dtensor=W, input_map=(1, -1, -1), forloop_dim=0)
    tM = tb.matmul(tX, tW)
    tO = tb.div(tb.forloop_accum(tM), tb.forloop_accum(tX, "rms"))
    tb.new_output(stensor=tO, output_map=(1, -1, -1))
    O_ = graph.customized([X, W], tb)
    graph.mark_output(O_[0], (4096, 1))
    opt = graph.superoptimize(backend="hip", profile_iters=0, use_graph_dataset=False)
    assert opt._plan.describe() == ["pack", "rmsnorm_linear"], opt._plan.describe()
    x = xs.cuda().t()
    w = ws.cuda().t()
    out = opt(inputs=[x, w])[0]
    torch.cuda.synchronize()
    xf = x.double().cpu()
    ref = (xf / torch.sqrt((xf * xf).mean(-1, keepdim=True) + 1e-6)).half().double() @ w.double().cpu()
    _close(out, ref.numpy(), "customized rmsnorm (column-major)")


@pytest.mark.parametrize("B", [8, 128])
def test_graph_gated_mlp(B):
    """BASELINE config 2a (B=8) and 2b (B=128, MFMA path), every column."""
    import yirage_amd.fused as F

    print(f"case graph gated MLP B={B}", flush=True)
    g = torch.Generator().manual_seed(0)
    K, N = 4096, 14336
    x = _randn((B, K), 1.0, torch.bfloat16, g)
    w1 = _randn((K, N), 0.02, torch.bfloat16, g)
    w3 = _randn((K, N), 0.02, torch.bfloat16, g)
    graph = yr.new_kernel_graph()
    X = graph.new_input(dims=(B, K), dtype=yr.bfloat16)
    W1 = graph.new_input(dims=(K, N), dtype=yr.bfloat16)
    W3 = graph.new_input(dims=(K, N), dtype=yr.bfloat16)
    graph.mark_output(graph.mul(graph.silu(graph.matmul(X, W1)), graph.matmul(X, W3)))
    opt = graph.superoptimize(backend="hip", warmup_iters=2, profile_iters=5, use_graph_dataset=False)
    assert opt._plan.describe() == ["gated_mlp"], opt._plan.describe()
    xc, w1c, w3c = x.cuda(), w1.cuda(), w3.cuda()
    out = opt(inputs=[xc, w1c, w3c])[0]
    direct = F.gated_mlp(xc, w1c, w3c)
    torch.cuda.synchronize()
    _same_bits(out, direct, "graph vs direct gated_mlp")
    O.set_num_threads(16)
    _close(out, O.gated_mlp(_f(x), _bits(w1), _bits(w3), "bf16", 1), f"graph gated_mlp B={B}")


def test_graph_gated_mlp_customized_demo():
    """demo/reference_mugraphs/gated_mlp.py / test_tensor_program.py:44-112."""
    print("case customized gated MLP", flush=True)
    g = torch.Generator().manual_seed(2)
    x = (torch.rand((8, 4096), generator=g) * -0.5 + 1).half()
    w1 = (torch.rand((4096, 4096), generator=g) * -0.5 + 1).half() * 0.01
    w2 = (torch.rand((4096, 4096), generator=g) * -0.5 + 1).half() * 0.01
    graph = yr.new_kernel_graph()
    X = graph.new_input(dims=(8, 4096), dtype=yr.float16)
    W1 = graph.new_input(dims=(4096, 4096), dtype=yr.float16)
    W2 = graph.new_input(dims=(4096, 4096), dtype=yr.float16)
    tb = yr.new_threadblock_graph(grid_dim=(64, 1, 1), block_dim=(128, 1, 1), forloop_range=32, reduction_dimx=64)
    tX = tb.new_input(dtensor=X, input_map=(-1, -1, -1), forloop_dim=1)
    tW1 = tb.new_input(dtensor=W1, input_map=(1, -1, -1), forloop_dim=0)
    tW2 = tb.new_input(dtensor=W2, input_map=(1, -1, -1), forloop_dim=0)
    tO = tb.mul(tb.silu(tb.forloop_accum(tb.matmul(tX, tW1))), tb.forloop_accum(tb.matmul(tX, tW2)))
    tb.new_output(stensor=tO, output_map=(1, -1, -1))
    O_ = graph.customized([X, W1, W2], tb)
    graph.mark_output(O_[0], (4096, 1))
    out = graph(inputs=[x.cuda(), w1.cuda(), w2.cuda()])[0]
    torch.cuda.synchronize()
    assert graph._plan.describe() == ["gated_mlp"]
    _close(out, O.gated_mlp(_f(x), _bits(w1), _bits(w2), "f16", 1), "customized gated MLP")


def _attention_graph(G, M, L, d, dt):
    graph = yr.new_kernel_graph()
    Q = graph.new_input(dims=(G, M, d), dtype=dt)
    K = graph.new_input(dims=(G, d, L), dtype=dt)
    V = graph.new_input(dims=(G, L, d), dtype=dt)
    E = graph.exp(graph.matmul(Q, K))
    graph.mark_output(graph.matmul(graph.div(E, graph.reduction(E, 2)), V))
    return graph


def _run_attention_op(q, k, v, out, G, M, L, d, scale):
    """The graph's attention step through yr_hip_run_fused with an explicit
    softmax scale (the graph itself always uses 1)."""
    dt = _lib.DTYPE_F16 if q.dtype == torch.float16 else _lib.DTYPE_BF16
    params = [G, M, L, d, dt, struct_bits(scale)] + list(q.stride()) + list(k.stride()) + list(v.stride()) + \
        list(out.stride())
    P = (ctypes.c_int64 * len(params))(*params)
    L_ = _lib.lib()
    nb = L_.yr_hip_fused_workspace(_lib.OP_ATTENTION, len(params), P)
    ws = torch.zeros(max(nb, 1), dtype=torch.uint8, device="cuda")
    ins = (ctypes.c_void_p * 3)(q.data_ptr(), k.data_ptr(), v.data_ptr())
    outs = (ctypes.c_void_p * 1)(out.data_ptr())
    _lib.check(L_.yr_hip_run_fused(_lib.OP_ATTENTION, 3, ins, 1, outs, len(params), P, ctypes.c_void_p(ws.data_ptr()),
                                   nb, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "attention")


def struct_bits(x):
    import struct
    return struct.unpack("<i", struct.pack("<f", x))[0]


def test_graph_attention_decode_shape_config3():
    """Config 3 shape as a kernel graph: 8 sequences x 8 kv heads = 64 groups
    of 4 query rows over 4096 keys.  The graph's attention step with the
    1/sqrt(d) scale is bit-identical to the paged decode kernel on the same
    data; the graph itself (unscaled softmax) matches the oracle."""
    import yirage_amd.fused as F

    print("case graph attention, config 3 shape", flush=True)
    gen = torch.Generator().manual_seed(0)
    B, Hq, Hkv, L, D, page = 8, 32, 8, 4096, 128, 64
    G = Hq // Hkv
    q = _randn((B, Hq, D), 1.0, torch.float16, gen)
    k = _randn((B, L, Hkv, D), 1.0, torch.float16, gen)
    v = _randn((B, L, Hkv, D), 1.0, torch.float16, gen)
    # paged form: page p of sequence b holds tokens 64 p .. 64 p + 63
    kc = k.view(B, L // page, page, Hkv, D).reshape(B * (L // page), page, Hkv, D).cuda()
    vc = v.view(B, L // page, page, Hkv, D).reshape(B * (L // page), page, Hkv, D).cuda()
    indptr = (torch.arange(B + 1, dtype=torch.int32) * (L // page)).cuda()
    indices = torch.arange(B * (L // page), dtype=torch.int32).cuda()
    lens = torch.full((B,), L, dtype=torch.int32).cuda()
    direct = F.gqa_decode_paged(q.cuda(), kc, vc, indptr, indices, lens, max_kv_len=L)
    # graph form: group = (sequence, kv head); K as the graph's [G][d][L]
    qg = q.view(B * Hkv, G, D).cuda()
    kg = k.permute(0, 2, 3, 1).reshape(B * Hkv, D, L).contiguous().cuda()
    vg = v.permute(0, 2, 1, 3).reshape(B * Hkv, L, D).contiguous().cuda()
    out = torch.empty_like(qg)
    _run_attention_op(qg, kg, vg, out, B * Hkv, G, L, D, 1.0 / math.sqrt(D))
    torch.cuda.synchronize()
    _same_bits(out.view(B, Hq, D), direct, "graph attention op vs paged decode")
    graph = _attention_graph(B * Hkv, G, L, D, yr.float16)
    got = graph(inputs=[qg, kg, vg])[0]
    torch.cuda.synchronize()
    assert graph._plan.describe() == ["attention"]
    # oracle: unscaled scores = (q sqrt(D)) . k / sqrt(D)
    ref = O.gqa_decode_paged(_f(q).astype(np.float64) * math.sqrt(D), _bits(kc.cpu()), _bits(vc.cpu()), "f16",
                             indptr.cpu().numpy(), indices.cpu().numpy(), lens.cpu().numpy())
    _close(got.view(B, Hq, D), ref, "graph attention (unscaled) config 3 shape")


def test_graph_attention_prefill_shape_config4():
    """Config 4 shape (S = 2048, 32 q / 8 kv heads) as a kernel graph,
    non-causal (the graph has no mask): the attention step with the 1/sqrt(d)
    scale is bit-identical to the prefill kernel; the unscaled graph output
    matches the oracle on a row sample of every head group."""
    import yirage_amd.fused as F

    print("case graph attention, config 4 shape", flush=True)
    gen = torch.Generator().manual_seed(0)
    S, Hq, Hkv, D = 2048, 32, 8, 128
    G = Hq // Hkv
    q = _randn((1, S, Hq, D), 1.0, torch.bfloat16, gen)
    k = _randn((1, S, Hkv, D), 1.0, torch.bfloat16, gen)
    v = _randn((1, S, Hkv, D), 1.0, torch.bfloat16, gen)
    direct = F.gqa_prefill(q.cuda(), k.cuda(), v.cuda(), causal=False)
    # group hk, row j S + s <- q[0, s, hk G + j]
    qg = q[0].view(S, Hkv, G, D).permute(1, 2, 0, 3).reshape(Hkv, G * S, D).contiguous().cuda()
    kg = k[0].permute(1, 2, 0).contiguous().cuda()          # [Hkv][D][S]
    vg = v[0].permute(1, 0, 2).contiguous().cuda()          # [Hkv][S][D]
    out = torch.empty_like(qg)
    _run_attention_op(qg, kg, vg, out, Hkv, G * S, S, D, 1.0 / math.sqrt(D))
    torch.cuda.synchronize()
    back = out.view(Hkv, G, S, D).permute(2, 0, 1, 3).reshape(1, S, Hq, D)
    _same_bits(back, direct, "graph attention op vs prefill")
    graph = _attention_graph(Hkv, G * S, S, D, yr.bfloat16)
    got = graph(inputs=[qg, kg, vg])[0]
    torch.cuda.synchronize()
    rows = [0, 1, 777, 2047]
    # float64 torch reference on sampled rows of every head
    kf, vf = k[0].double(), v[0].double()
    for r in rows:
        for h in range(Hq):
            hk = h // G
            s = (kf[:, hk] @ q[0, r, h].double())
            p = torch.softmax(s, 0)
            o = p @ vf[:, hk]
            g_row = got[hk, (h % G) * S + r].double().cpu()
            err = (g_row - o).abs()
            assert (err <= ATOL + RTOL * o.abs()).all(), f"row {r} head {h}: max err {err.max()}"
    print("[graph attention config 4 shape] sampled rows match", flush=True)


def test_graph_attention_reference_benchmark_shape():
    """benchmark/group_query_attention.py:37-46 at bs 1: Q (2, 256, 64),
    K (2, 64, 4096), V (2, 4096, 64), d = 64 (padded to 128 internally),
    and the two-customized-op form of demo/reference_mugraphs/
    group_query_attention.py on the same inputs."""
    print("case graph attention, reference benchmark shape (d = 64)", flush=True)
    gen = torch.Generator().manual_seed(3)
    q = (torch.randn((2, 256, 64), generator=gen) * 0.2 - 0.1).half()
    k = (torch.randn((2, 64, 4096), generator=gen) * 0.2 - 0.1).half()
    v = (torch.randn((2, 4096, 64), generator=gen) * 0.2 - 0.1).half()
    ref = torch.softmax(q.double() @ k.double(), -1) @ v.double()
    graph = _attention_graph(2, 256, 4096, 64, yr.float16)
    opt = graph.superoptimize(backend="hip", warmup_iters=1, profile_iters=3, use_graph_dataset=False)
    got = opt(inputs=[q.cuda(), k.cuda(), v.cuda()])[0]
    torch.cuda.synchronize()
    _close(got, ref.numpy(), "graph attention d=64")
    # customized two-op form
    g2 = yr.new_kernel_graph()
    Q = g2.new_input(dims=(2, 256, 64), dtype=yr.float16)
    K = g2.new_input(dims=(2, 64, 4096), dtype=yr.float16)
    V = g2.new_input(dims=(2, 4096, 64), dtype=yr.float16)
    t1 = yr.new_threadblock_graph(grid_dim=(2, 16, 4), block_dim=(128, 1, 1), forloop_range=4, reduction_dimx=64)
    bQ = t1.new_input(dtensor=Q, input_map=(0, -1, 1), forloop_dim=-1)
    bK = t1.new_input(dtensor=K, input_map=(0, 2, -1), forloop_dim=2)
    bV = t1.new_input(dtensor=V, input_map=(0, 1, -1), forloop_dim=1)
    bE = t1.exp(t1.matmul(bQ, bK))
    t1.new_output(stensor=t1.forloop_accum(t1.matmul(bE, bV)), output_map=(0, 2, 1))
    t1.new_output(stensor=t1.forloop_accum(bE, "sum"), output_map=(0, 2, 1))
    O1 = g2.customized([Q, K, V], t1)
    t2 = yr.new_threadblock_graph(grid_dim=(2, 16, 1), block_dim=(128, 1, 1), forloop_range=1, reduction_dimx=64)
    bA = t2.forloop_accum(t2.new_input(dtensor=O1[0], input_map=(0, 1, -1), forloop_dim=-1), "sum_todimx")
    bB = t2.forloop_accum(t2.new_input(dtensor=O1[1], input_map=(0, 1, -1), forloop_dim=-1), "sum")
    t2.new_output(stensor=t2.div(bA, bB), output_map=(0, 1, -1))
    O2 = g2.customized(O1, t2)
    g2.mark_output(O2[0], (256 * 64, 64, 1))
    got2 = g2(inputs=[q.cuda(), k.cuda(), v.cuda()])[0]
    torch.cuda.synchronize()
    assert g2._plan.describe() == ["attention"]
    # (superoptimize keeps whichever plan measured faster; the fused plan
    # of the kernel graph is the one the two-op form must equal bit for bit)
    fused = graph._execute(graph.plan(fuse=True), [q.cuda(), k.cuda(), v.cuda()], None)[0]
    torch.cuda.synchronize()
    _same_bits(got2, fused, "customized GQA vs kernel-graph GQA")


def _round(x, dt):
    return x.to(dt).double()


def test_graph_generic_ops_norm_transformer():
    """benchmark/norm_transformer.py:38-46: rms_norm, add, mul, add, rms_norm
    -- no fused pattern, every op on its generic HIP kernel."""
    print("case generic ops: norm_transformer", flush=True)
    gen = torch.Generator().manual_seed(4)
    dt = torch.float16
    B = 16
    h, x, alpha = (_randn((B, 4096), 1.0, dt, gen) for _ in range(3))
    graph = yr.new_kernel_graph()
    H = graph.new_input(dims=(B, 4096), dtype=yr.float16)
    X = graph.new_input(dims=(B, 4096), dtype=yr.float16)
    A = graph.new_input(dims=(B, 4096), dtype=yr.float16)
    C = graph.add(X, graph.mul(A, graph.add(graph.rms_norm(H, normalized_shape=(4096,)), X)))
    graph.mark_output(graph.rms_norm(C, normalized_shape=(4096,)))
    opt = graph.superoptimize(backend="hip", profile_iters=0, use_graph_dataset=False)
    # the add-mul-add tree runs as one fused elementwise launch
    assert opt._plan.describe() == ["rms_norm", "ewise(add+mul+add)", "rms_norm"]
    got = opt(inputs=[h.cuda(), x.cuda(), alpha.cuda()])[0]
    torch.cuda.synchronize()

    def rms(t):
        return _round(t / torch.sqrt((t * t).mean(-1, keepdim=True) + 1e-6), dt)
    hd, xd, ad = h.double(), x.double(), alpha.double()
    c = _round(xd + _round(ad * _round(rms(hd) + xd, dt), dt), dt)
    _close(got, rms(c).numpy(), "norm_transformer")


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_graph_generic_matmul_elementwise_reduction(dt):
    """Batched matmul (MFMA), unary ops with broadcasting binaries and a
    reduction over a middle dim, on shapes with ragged tiles."""
    print(f"case generic ops: matmul / elementwise / reduction {dt}", flush=True)
    gen = torch.Generator().manual_seed(5)
    a = _randn((3, 100, 72), 0.3, dt, gen)
    b = _randn((3, 72, 136), 0.3, dt, gen)
    c = _randn((3, 1, 136), 1.0, dt, gen)
    ydt = yr.float16 if dt == torch.float16 else yr.bfloat16
    graph = yr.new_kernel_graph()
    A = graph.new_input(dims=(3, 100, 72), dtype=ydt)
    Bm = graph.new_input(dims=(3, 72, 136), dtype=ydt)
    Cb = graph.new_input(dims=(3, 1, 136), dtype=ydt)
    M = graph.matmul(A, Bm)
    T = graph.gelu(graph.add(M, Cb))
    graph.mark_output(M)
    graph.mark_output(graph.reduction(graph.square(T), 1))
    graph.mark_output(graph.clamp(graph.div(T, Cb), -0.5, 0.5))
    outs = graph(inputs=[a.cuda(), b.cuda(), c.cuda()])
    torch.cuda.synchronize()
    # single-consumer elementwise chains run as fused elementwise launches
    assert graph._plan.describe() == ["matmul", "ewise(add+gelu)", "square", "reduction", "ewise(div+clamp)"]
    m = _round(a.double() @ b.double(), dt)
    t = _round(torch.nn.functional.gelu(_round(m + c.double(), dt)), dt)
    _close(outs[0], m.numpy(), "matmul")
    r = _round(_round(t * t, dt).sum(1, keepdim=True), dt)
    _close(outs[1], r.numpy(), "square + reduction", rtol=2e-2, atol=2e-2)
    _close(outs[2], _round(torch.clamp(_round(t / c.double(), dt), -0.5, 0.5), dt).numpy(), "div + clamp")


def test_superoptimize_profiles_and_caches():
    """The hip branch of superoptimize profiles its candidates, returns a
    graph bound to the faster plan and stores it in graph_dataset."""
    print("case superoptimize cache", flush=True)
    yr.graph_dataset.clear()
    graph = yr.new_kernel_graph()
    X = graph.new_input(dims=(8, 1024), dtype=yr.float16)
    W = graph.new_input(dims=(1024, 512), dtype=yr.float16)
    graph.mark_output(graph.matmul(graph.rms_norm(X, normalized_shape=(1024,)), W))
    g1 = graph.superoptimize(backend="hip", warmup_iters=2, profile_iters=10, verbose=True)
    g2 = graph.superoptimize(backend="hip", warmup_iters=2, profile_iters=10)
    assert g1 is g2 and g1.backend == "hip"
    gen = torch.Generator().manual_seed(6)
    x = _randn((8, 1024), 1.0, torch.float16, gen)
    w = _randn((1024, 512), 0.05, torch.float16, gen)
    out = g1(inputs=[x.cuda(), w.cuda()])[0]
    torch.cuda.synchronize()
    _close(out, O.rmsnorm_linear(_f(x), None, _bits(w), "f16", 1, 1e-6), "superoptimized")
