"""CPU checks of the kernel-graph front end (no GPU): shape rules of the
reference's kernel / threadblock ops, the pattern matcher's plans for the
graphs the reference's benchmarks and demos build, the structural hash, the
graph-dataset cache and the C ABI's workspace queries for graph steps."""
import pytest

import yirage_amd as yr
from yirage_amd import YirageHipError, _lib


def _rms_linear(B=8, K=4096, N=4096, gamma=False):
    g = yr.new_kernel_graph()
    X = g.new_input(dims=(B, K), dtype=yr.float16)
    W = g.new_input(dims=(K, N), dtype=yr.float16)
    D = g.rms_norm(X, normalized_shape=(K,))
    if gamma:
        G = g.new_input(dims=(1, K), dtype=yr.float16)
        D = g.mul(D, G)
    g.mark_output(g.matmul(D, W))
    return g


def _attention(G=2, M=256, L=4096, d=64, div_last=False):
    g = yr.new_kernel_graph()
    Q = g.new_input(dims=(G, M, d), dtype=yr.float16)
    K = g.new_input(dims=(G, d, L), dtype=yr.float16)
    V = g.new_input(dims=(G, L, d), dtype=yr.float16)
    E = g.exp(g.matmul(Q, K))
    S = g.reduction(E, 2)
    O = g.div(g.matmul(E, V), S) if div_last else g.matmul(g.div(E, S), V)
    g.mark_output(O)
    return g


def test_shape_rules():
    g = yr.new_kernel_graph()
    A = g.new_input(dims=(2, 16, 32), dtype=yr.bfloat16)
    B = g.new_input(dims=(2, 32, 8), dtype=yr.bfloat16)
    C = g.matmul(A, B)
    assert C.dims == (2, 16, 8) and C.dtype == yr.bfloat16
    assert g.reduction(C, 1).dims == (2, 1, 8)
    bias = g.new_input(dims=(1, 1, 8), dtype=yr.bfloat16)
    assert g.add(C, bias).dims == (2, 16, 8)
    assert g.rms_norm(C, normalized_shape=(8,)).dims == (2, 16, 8)
    with pytest.raises(ValueError):
        g.matmul(A, A)                       # inner dims 32 != 16
    with pytest.raises(ValueError):
        g.add(C, g.new_input(dims=(2, 3, 8), dtype=yr.bfloat16))
    with pytest.raises(ValueError):
        g.rms_norm(C, normalized_shape=(16,))
    with pytest.raises(AssertionError):
        g.new_input(dims=(4, 4), strides=(4, 2))  # neither row- nor column-major


def test_threadblock_shapes_of_the_gqa_demo():
    """demo/reference_mugraphs/group_query_attention.py: the two customized
    ops' output dims follow input_map / output_map / forloop rules."""
    g = yr.new_kernel_graph()
    Q = g.new_input(dims=(2, 256, 64), dtype=yr.float16)
    K = g.new_input(dims=(2, 64, 4096), dtype=yr.float16)
    V = g.new_input(dims=(2, 4096, 64), dtype=yr.float16)
    t1 = yr.new_threadblock_graph(grid_dim=(2, 16, 4), block_dim=(128, 1, 1), forloop_range=4, reduction_dimx=64)
    bQ = t1.new_input(dtensor=Q, input_map=(0, -1, 1), forloop_dim=-1)
    bK = t1.new_input(dtensor=K, input_map=(0, 2, -1), forloop_dim=2)
    bV = t1.new_input(dtensor=V, input_map=(0, 1, -1), forloop_dim=1)
    assert (bQ.dims, bK.dims, bV.dims) == ((1, 64, 64), (1, 64, 64), (1, 64, 64))
    bE = t1.exp(t1.matmul(bQ, bK))
    t1.new_output(stensor=t1.forloop_accum(t1.matmul(bE, bV)), output_map=(0, 2, 1))
    t1.new_output(stensor=t1.forloop_accum(bE, "sum"), output_map=(0, 2, 1))
    O1 = g.customized([Q, K, V], t1)
    assert [o.dims for o in O1] == [(2, 256, 1024), (2, 256, 16)]
    t2 = yr.new_threadblock_graph(grid_dim=(2, 16, 1), block_dim=(128, 1, 1), forloop_range=1, reduction_dimx=64)
    bA = t2.forloop_accum(t2.new_input(dtensor=O1[0], input_map=(0, 1, -1), forloop_dim=-1), "sum_todimx")
    bB = t2.forloop_accum(t2.new_input(dtensor=O1[1], input_map=(0, 1, -1), forloop_dim=-1), "sum")
    assert bA.dims == (1, 16, 64) and bB.dims == (1, 16, 1)
    t2.new_output(stensor=t2.div(bA, bB), output_map=(0, 1, -1))
    O2 = g.customized(O1, t2)
    assert O2[0].dims == (2, 256, 64)
    g.mark_output(O2[0])
    assert g.plan().describe() == ["attention"]


def test_plans_of_the_hot_patterns():
    assert _rms_linear().plan().describe() == ["rmsnorm_linear"]
    assert _rms_linear(gamma=True).plan().describe() == ["rmsnorm_linear"]
    assert _rms_linear().plan(fuse=False).describe() == ["rms_norm", "matmul"]
    assert _attention().plan().describe() == ["attention"]
    assert _attention(div_last=True).plan().describe() == ["attention"]
    assert _attention().plan(fuse=False).describe() == ["matmul", "exp", "reduction", "div", "matmul"]
    g = yr.new_kernel_graph()
    X = g.new_input(dims=(8, 4096), dtype=yr.bfloat16)
    W1 = g.new_input(dims=(4096, 14336), dtype=yr.bfloat16)
    W3 = g.new_input(dims=(4096, 14336), dtype=yr.bfloat16)
    g.mark_output(g.mul(g.matmul(X, W3), g.silu(g.matmul(X, W1))))  # operands swapped
    p = g.plan()
    assert p.describe() == ["gated_mlp"]
    assert p.steps[0].params == [8, 4096, 14336, 941, _lib.W_KN]


def test_fusion_respects_other_consumers():
    """An intermediate that is also a graph output (or feeds another op)
    cannot disappear into a fused kernel."""
    g = yr.new_kernel_graph()
    X = g.new_input(dims=(8, 1024), dtype=yr.float16)
    W = g.new_input(dims=(1024, 512), dtype=yr.float16)
    D = g.rms_norm(X, normalized_shape=(1024,))
    g.mark_output(g.matmul(D, W))
    g.mark_output(D)
    assert g.plan().describe() == ["rms_norm", "linear"]


def test_column_major_weight_is_nk_and_linear_residual():
    g = yr.new_kernel_graph()
    X = g.new_input(dims=(4, 1024), dtype=yr.float16)
    W = g.new_input(dims=(1024, 512), strides=(1, 1024), dtype=yr.float16)  # stored N x K
    R = g.new_input(dims=(4, 512), dtype=yr.float16)
    g.mark_output(g.add(g.matmul(X, W), R))
    p = g.plan()
    assert p.describe() == ["linear_residual"]
    assert p.steps[0].params == [4, 1024, 512, 940, _lib.W_NK]
    assert p.steps[0].ins == [("in", 0), ("in", 1), ("in", 2)] and p.steps[0].outs == [("out", 0)]


def test_strided_output_gets_a_pack_step():
    g = _rms_linear(B=8, K=1024, N=512)
    t, _ = g.outputs[0]
    g.outputs[0] = (t, (1, 8))  # column-major output
    assert g.plan().describe() == ["rmsnorm_linear", "pack_output"]


def test_unsupported_customized_graph_raises():
    g = yr.new_kernel_graph()
    X = g.new_input(dims=(8, 64), dtype=yr.float16)
    # a rescale tile with one factor per element instead of per row (the
    # reference's rescale kernel rejects it too): no fused kernel, no
    # whole-tensor expression and no generic form
    tb = yr.new_threadblock_graph(grid_dim=(1, 1, 1), block_dim=(128, 1, 1), forloop_range=2, reduction_dimx=64)
    tX = tb.new_input(dtensor=X, input_map=(-1, -1, -1), forloop_dim=1)
    tb.new_output(stensor=tb.forloop_accum_rescale(tb.exp(tX), tX), output_map=(-1, -1, -1))
    g.mark_output(g.customized([X], tb)[0])
    with pytest.raises(YirageHipError):
        g.plan()


def test_owner_independent_hash():
    assert _rms_linear().get_owner_independent_hash() == _rms_linear().get_owner_independent_hash()
    assert _rms_linear().get_owner_independent_hash() != _rms_linear(B=16).get_owner_independent_hash()
    assert _attention().get_owner_independent_hash() != _attention(div_last=True).get_owner_independent_hash()


def test_superoptimize_without_gpu_caches_and_rejects_other_backends():
    yr.graph_dataset.clear()
    g = _rms_linear()
    o1 = g.superoptimize(backend="hip", profile_iters=0)
    o2 = _rms_linear().superoptimize(backend="hip", profile_iters=0)  # same structure: cache hit
    assert o1 is o2 and o1.backend == "hip" and o1._plan.describe() == ["rmsnorm_linear"]
    o3 = _rms_linear().superoptimize(backend="hip", profile_iters=0, griddims=[(64, 1, 1)])
    assert o3 is not o1  # different search arguments: a separate entry
    with pytest.raises(YirageHipError):
        g.superoptimize(backend="cuda")


def test_graph_step_workspace_queries():
    """Workspace sizes of graph steps come from the C ABI (no GPU)."""
    p = _attention(G=2, M=256, L=4096, d=64).plan()
    assert p.workspace_bytes() > 64 * 1024          # packed K^T -> K and padded Q / V / O
    p = _attention(G=64, M=4, L=4096, d=128).plan()
    assert p.workspace_bytes() > 64 * 1024          # split-KV decode records + packed K
    p = _rms_linear().plan()
    assert p.workspace_bytes() == _lib.lib().yr_hip_rmsnorm_linear_workspace(8, 4096, 4096, 940, _lib.W_KN)
    L = _lib.lib()
    import ctypes
    bad = (ctypes.c_int64 * 2)(1, 2)
    assert L.yr_hip_fused_workspace(99, 2, bad) == 0
    rc = L.yr_hip_run_fused(_lib.OP_BINARY, 2, None, 1, None, 2, bad, None, 0, None)
    assert rc == -1


def test_checkpoint_written_under_the_looked_up_name(tmp_path, monkeypatch):
    """save_codes=True writes the candidate list as
    yirage_cached_mugraphs_<hash>.json; a later superoptimize() of the same
    structure (graph-dataset cache off) reads it back as a candidate."""
    import json as _json

    from yirage_amd import mugraph_json

    monkeypatch.chdir(tmp_path)
    g = _rms_linear()
    name = f"yirage_cached_mugraphs_{g.get_owner_independent_hash():x}.json"
    g.superoptimize(backend="hip", profile_iters=0, use_graph_dataset=False, save_codes=True)
    assert (tmp_path / name).exists()
    saved = mugraph_json.load(str(tmp_path / name))
    assert len(saved) == 1 and g._same_interface(saved[0])
    assert saved[0].plan(fuse=True).describe() == g.plan(fuse=True).describe()
    assert isinstance(_json.loads((tmp_path / name).read_text())[0], list)
    g2 = _rms_linear().superoptimize(backend="hip", profile_iters=0, use_graph_dataset=False)
    assert g2._plan.describe() == g.plan(fuse=True).describe()
