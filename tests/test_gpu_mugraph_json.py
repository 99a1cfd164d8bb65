"""GPU parity of the candidates the reference's search saved
(tests/golden/saved_mugraphs/: benchmark/saved_mugraphs/{cuda,mps}/*.json and
tests/ci-tests/qwen2.5/mirage_cached_mugraphs_*.json as shipped), loaded with
yirage_amd.mugraph_json and run on the hip backend.  Each file's graphs are
different factorizations of one computation; every plannable candidate
(in files with more than 8: the first, a middle, the last and the first of
each distinct plan) is checked
against the CPU oracle (RMSNorm + linear, gated MLP, linear, silu-mul) or a
float64 torch restatement of the benchmark's graph (softmax attention,
LoRA, the norm-transformer block: candidates the fused patterns do not
cover run as generic steps, or literally, tile by tile) or, for the saved
qk-norm candidates, a block-by-block numpy emulation of their own
threadblock graphs, within rtol/atol 1e-2 (the tolerance of the reference's
tests/python/test_tensor_program.py; atol 1e-3 for attention, whose outputs
are averages of order 0.1)."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from yirage_amd import YirageHipError
from yirage_amd import mugraph_json as MJ

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "saved_mugraphs")
RTOL, ATOL = 1e-2, 1e-2


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _inputs(g, stds, seed):
    """Device tensors with each input's dims and strides (a column-major
    weight is the transpose of a contiguous [N, K] tensor)."""
    gen = torch.Generator().manual_seed(seed)
    out = []
    for t, std in zip(g.inputs, stds):
        n = sum((d - 1) * s for d, s in zip(t.dims, t.strides)) + 1
        base = (torch.randn(n, generator=gen) * std).to(t.dtype.torch)
        out.append(torch.as_strided(base, t.dims, t.strides))
    return out


def _reference(kind, g, ins):
    dt = "f16" if g.inputs[0].dtype.torch == torch.float16 else "bf16"
    if kind == "attention":
        q, k, v = (x.double() for x in ins)
        return (torch.softmax(q @ k, -1) @ v).numpy()
    if kind == "linear":
        x, W = ins
        return O.linear(x.float().numpy(), _bits(W), dt, O.W_KN)
    if kind == "rmsnorm":
        x, W = ins
        return O.rmsnorm_linear(x.float().numpy(), None, _bits(W), dt, O.W_KN)
    if kind == "rmsnorm_gamma_nk":
        x, gm, W = ins
        return O.rmsnorm_linear(x.float().numpy(), gm.float().numpy().reshape(-1), _bits(W.t()), dt, O.W_NK)
    if kind == "gated":
        x, W1, W3 = ins
        return O.gated_mlp(x.float().numpy(), _bits(W1), _bits(W3), dt, O.W_KN)
    if kind == "silu_mul_linear_nk":
        a, u, W = ins
        h = O.silu_mul(a.float().numpy(), u.float().numpy(), dt)
        return O.linear(h, _bits(W.t()), dt, O.W_NK)
    if kind == "lora":
        # benchmark/lora.py: O = X W + (X A) B
        x, W, A, B = (t.double() for t in ins)
        return (x @ W + (x @ A) @ B).numpy()
    if kind == "emulate":
        # the graph's own threadblock semantics, block by block (tests/tb_numpy.py)
        from tb_numpy import run_graph
        return run_graph(g, [t.double().numpy() for t in ins])[0]
    if kind == "ntrans":
        # benchmark/norm_transformer.py: O = rms_norm(X + alpha (rms_norm(H) + X))
        H, x, alpha = (t.double() for t in ins)

        def rms(t):
            return t / torch.sqrt((t * t).mean(-1, keepdim=True) + 1e-6)
        return rms(x + alpha * (rms(H) + x)).numpy()
    raise AssertionError(kind)


CASES = [
    # file, reference, input stds
    ("rmsnorm_bs1.json", "rmsnorm", (1.0, 0.02)),
    ("mirage_cached_mugraphs_647dd41aeaf656b4.json", "rmsnorm_gamma_nk", (1.0, 1.0, 0.02)),
    ("mirage_cached_mugraphs_64644b2e7bbffb94.json", "silu_mul_linear_nk", (1.0, 1.0, 0.01)),
    ("single_gated_mlp.json", "gated", (1.0, 0.02, 0.02)),
    ("mps_yirage_cached_mugraphs_7310eff92c865e30.json", "linear", (1.0, 0.1)),
    ("gqa_bs8.json", "attention", (0.5, 0.5, 1.0)),
    ("single_mqa_bs1.json", "attention", (0.5, 0.5, 1.0)),
    # one MHA candidate runs the graph literally (generic steps: exp without
    # max subtraction, fp16 row sums), so scores stay small enough for fp16
    ("mha_bs1.json", "attention", (0.25, 0.25, 1.0)),
    ("single_lora.json", "lora", (1.0, 0.05, 0.05, 0.25)),
    ("ntrans_bs1.json", "ntrans", (1.0, 1.0, 1.0)),
    # the saved qk-norm candidates do not compute the function of
    # benchmark/qknorm_gqa.py's graph (block-by-block emulations of the two
    # differ; the candidates agree with one another): they are checked
    # against their own threadblock semantics
    ("qknorm_gqa_bs1_subset.json", "emulate", (1.0, 0.02, 1.0)),  # K small: the literal fp16 row sums stay finite
]


@pytest.mark.parametrize("name,kind,stds", CASES, ids=[c[0] for c in CASES])
def test_saved_candidates_match_the_oracle(name, kind, stds):
    gs = MJ.load(os.path.join(GOLDEN, name))
    plannable = []
    for i, g in enumerate(gs):
        try:
            g.plan(fuse=True)
        except YirageHipError:
            continue
        plannable.append(i)
    assert plannable
    if len(plannable) <= 8:
        pick = plannable
    else:  # first, middle, last, and the first of every distinct plan
        first_of = {}
        for i in plannable:
            first_of.setdefault(tuple(gs[i].plan(fuse=True).describe()), i)
        pick = sorted({plannable[0], plannable[len(plannable) // 2], plannable[-1], *first_of.values()})
    ins = _inputs(gs[pick[0]], stds, seed=len(name))
    ref = _reference(kind, gs[pick[0]], ins) if kind != "emulate" else None
    dev = [x.cuda() for x in ins]  # dense views keep their strides
    assert all(d.stride() == t.strides for d, t in zip(dev, gs[pick[0]].inputs))
    for i in pick:
        g = gs[i]
        print(f"case {name} candidate {i} plan {g.plan(fuse=True).describe()}", flush=True)
        got = g(inputs=dev)[0]
        torch.cuda.synchronize()
        if kind == "emulate":
            ref = _reference(kind, g, ins)
        err = np.abs(got.float().cpu().numpy() - ref)
        # attention outputs average thousands of V rows (|o| ~ 0.1): a tighter atol
        atol = 1e-3 if kind == "attention" else ATOL
        bad = err > atol + RTOL * np.abs(ref)
        print(f"[{name} #{i}] max abs err {err.max():.3e}, mismatches {bad.sum()}/{bad.size}", flush=True)
        assert not bad.any(), f"{name} candidate {i}: {bad.sum()} elements outside rtol/atol"


def test_customized_whole_tensor_expression_matches_torch():
    """A customized op that no fused pattern covers, lowered to generic
    steps: exp over a 2 x 2 grid of tiles, placed back where they came from,
    equals torch.exp of the whole tensor (fp16 rounding)."""
    import yirage_amd as yr

    g = yr.new_kernel_graph()
    X = g.new_input(dims=(64, 64), dtype=yr.float16)
    tb = yr.new_threadblock_graph(grid_dim=(2, 2, 1), block_dim=(128, 1, 1), forloop_range=1, reduction_dimx=64)
    tX = tb.new_input(dtensor=X, input_map=(0, 1, -1), forloop_dim=-1)
    tb.new_output(stensor=tb.forloop_accum(tb.exp(tX)), output_map=(0, 1, -1))
    g.mark_output(g.customized([X], tb)[0])
    x = (torch.randn((64, 64), generator=torch.Generator().manual_seed(1))).half()
    got = g(inputs=[x.cuda()])[0]
    torch.cuda.synchronize()
    assert g._plan.describe() == ["exp"]
    ref = torch.exp(x.double()).numpy()
    err = np.abs(got.float().cpu().numpy() - ref)
    assert not (err > ATOL + RTOL * np.abs(ref)).any(), f"max err {err.max()}"


def test_customized_block_transpose_runs_literally():
    """A customized op whose output map puts each block's tile at the
    transposed block position is no whole-tensor expression: it runs tile by
    tile (gather, exp, scatter) and must equal exp of X with its 32 x 32
    blocks swapped across the diagonal."""
    import yirage_amd as yr

    g = yr.new_kernel_graph()
    X = g.new_input(dims=(64, 64), dtype=yr.float16)
    tb = yr.new_threadblock_graph(grid_dim=(2, 2, 1), block_dim=(128, 1, 1), forloop_range=1, reduction_dimx=64)
    tX = tb.new_input(dtensor=X, input_map=(0, 1, -1), forloop_dim=-1)
    tb.new_output(stensor=tb.forloop_accum(tb.exp(tX)), output_map=(1, 0, -1))
    g.mark_output(g.customized([X], tb)[0])
    x = (torch.randn((64, 64), generator=torch.Generator().manual_seed(2))).half()
    got = g(inputs=[x.cuda()])[0]
    torch.cuda.synchronize()
    assert g._plan.describe() == ["copy_nd", "exp", "copy_nd"]
    prog = g.plan(fuse=True, tb_program=True)
    assert prog.describe() == ["tb_program"]
    got_prog = g._execute(prog, [x.cuda()], None)[0]
    torch.cuda.synchronize()
    e = torch.exp(x.double())
    ref = e.view(2, 32, 2, 32).permute(2, 1, 0, 3).reshape(64, 64).numpy()  # block (i, j) -> (j, i)
    for out in (got, got_prog):
        err = np.abs(out.float().cpu().numpy() - ref)
        assert not (err > ATOL + RTOL * np.abs(ref)).any(), f"max err {err.max()}"
    assert torch.equal(got, got_prog)  # one exp, one rounding either way


def _run(g, ins, tbp):
    """g's plan with its customized ops run literally or as tile programs."""
    p = g.plan(fuse=True, tb_program=tbp)
    assert ("tb_program" in p.describe()) == tbp, p.describe()
    out = g._execute(p, [x.cuda() for x in ins], None)
    torch.cuda.synchronize()
    return out


def test_customized_unary_chain_as_tile_program():
    """Every unary kind (silu, gelu, relu, clamp, square, sqrt, mul_scalar,
    exp) and add / div in one block-transposed customized op, run as a tile
    program and literally, against float64 torch (each operator's result is
    rounded to fp16 in both plans, hence the tolerance)."""
    import yirage_amd as yr

    g = yr.new_kernel_graph()
    X = g.new_input(dims=(64, 64), dtype=yr.float16)
    tb = yr.new_threadblock_graph(grid_dim=(2, 2, 1), block_dim=(128, 1, 1), forloop_range=1, reduction_dimx=64)
    t = tb.new_input(dtensor=X, input_map=(0, 1, -1), forloop_dim=-1)
    s = tb.add(tb.silu(t), tb.gelu(t))
    s = tb.add(s, tb.relu(t))
    s = tb.add(s, tb.clamp(t, -0.5, 0.5))
    s = tb.add(s, tb.sqrt(tb.square(t)))
    s = tb.add(s, tb.mul_scalar(t, 0.5))
    s = tb.div(s, tb.exp(t))
    tb.new_output(stensor=tb.forloop_accum(s), output_map=(1, 0, -1))
    g.mark_output(g.customized([X], tb)[0])
    x = (torch.randn((64, 64), generator=torch.Generator().manual_seed(9))).half()
    xd = x.double()
    ref = (torch.nn.functional.silu(xd) + torch.nn.functional.gelu(xd) + torch.relu(xd) + xd.clamp(-0.5, 0.5)
           + xd.abs() + 0.5 * xd) / torch.exp(xd)
    ref = ref.view(2, 32, 2, 32).permute(2, 1, 0, 3).reshape(64, 64).numpy()
    for tbp in (True, False):
        got = _run(g, [x], tbp)[0]
        err = np.abs(got.float().cpu().numpy() - ref)
        assert not (err > 2 * ATOL + 2 * RTOL * np.abs(ref)).any(), f"tile program {tbp}: max err {err.max()}"


@pytest.mark.parametrize("tbp", [False, True], ids=["literal", "tile_program"])
def test_customized_max_and_concat_run_literally(tbp):
    """Forloop max accumulator, reduction_max and concat on the GPU against
    the block-by-block emulation (tests/tb_numpy.py), run literally and as a
    tile program."""
    from tb_numpy import run_graph
    from test_mugraph_json import _max_concat_graph

    g = _max_concat_graph()
    x = (torch.randn((8, 256), generator=torch.Generator().manual_seed(4))).half()
    got = _run(g, [x], tbp)[0]
    ref = run_graph(g, [x.double().numpy()])[0]
    err = np.abs(got.float().cpu().numpy() - ref)
    assert not (err > ATOL + RTOL * np.abs(ref)).any(), f"max err {err.max()}"


@pytest.mark.parametrize("tbp", [False, True], ids=["literal", "tile_program"])
def test_customized_mean_accumulator_runs_literally(tbp):
    """The mean forloop accumulator on the GPU against its closed form, the
    row mean of exp(X) (float64), and the sum accumulator of the same tiles
    divided by the 256 summed elements; literally and as a tile program."""
    from test_mugraph_json import _mean_graph

    g = _mean_graph()
    x = (torch.randn((8, 256), generator=torch.Generator().manual_seed(5))).half()
    mean, total = _run(g, [x], tbp)
    ref = torch.exp(x.double()).mean(1, keepdim=True).numpy()
    err = np.abs(mean.float().cpu().numpy() - ref)
    assert not (err > ATOL + RTOL * np.abs(ref)).any(), f"max err {err.max()}"
    err2 = np.abs(mean.float().cpu().numpy() - total.float().cpu().numpy() / 256)
    assert not (err2 > ATOL + RTOL * np.abs(ref)).any(), f"mean vs sum / 256: {err2.max()}"


@pytest.mark.parametrize("tbp", [False, True], ids=["literal", "tile_program"])
def test_customized_rescale_accumulator_runs_literally(tbp):
    """Rescale accumulators (acc = acc * rescale + input per iteration, kept
    whole and with the last dim summed) on the GPU against the closed form
    sum_i x_i prod_{j>i} r_j in float64; literally and as a tile program."""
    from test_mugraph_json import _rescale_closed_form, _rescale_graph

    g = _rescale_graph()
    x = (torch.randn((8, 256), generator=torch.Generator().manual_seed(7))).half()
    whole, summed = _run(g, [x], tbp)
    want, want_sum = _rescale_closed_form(x.double().numpy())
    for got, ref in ((whole, want), (summed, want_sum)):
        err = np.abs(got.float().cpu().numpy() - ref)
        assert not (err > ATOL + RTOL * np.abs(ref)).any(), f"max err {err.max()}"


@pytest.mark.parametrize("name,kind,stds", [c for c in CASES if c[0] in ("mha_bs1.json", "ntrans_bs1.json",
                                                                          "qknorm_gqa_bs1_subset.json")],
                         ids=["mha", "ntrans", "qknorm"])
def test_tile_programs_match_the_literal_plans(name, kind, stds):
    """Every saved candidate whose customized op runs as a tile program
    (yr_hip_tb_program, one launch) against the same graph run literally
    (one launch per threadblock op, block tensors in HBM) and against the
    block-by-block float64 emulation (tests/tb_numpy.py), on the GPU."""
    from tb_numpy import run_graph

    gs = MJ.load(os.path.join(GOLDEN, name))
    checked = 0
    for i, g in enumerate(gs):
        try:
            pt = g.plan(fuse=True, tb_program=True)
            pl = g.plan(fuse=True)
        except YirageHipError:
            continue
        if "tb_program" not in pt.describe():
            continue
        print(f"case {name} candidate {i}: {pt.describe()}", flush=True)
        ins = _inputs(g, stds, seed=i)
        dev = [x.cuda() for x in ins]
        a = g._execute(pt, dev, None)[0]
        b = g._execute(pl, dev, None)[0]
        torch.cuda.synchronize()
        ref = run_graph(g, [x.double().numpy() for x in ins])[0]
        for out, what in ((a, "tile program"), (b, "literal plan")):
            err = np.abs(out.float().cpu().numpy() - ref)
            atol = 1e-3 if kind == "attention" else ATOL
            bad = err > atol + RTOL * np.abs(ref)
            assert not bad.any(), f"{name} candidate {i} ({what}): {bad.sum()} outside, max err {err.max()}"
        checked += 1
    assert checked >= {"mha_bs1.json": 15, "ntrans_bs1.json": 3, "qknorm_gqa_bs1_subset.json": 12}[name]


def test_superoptimize_times_tile_program_candidates(capsys):
    """superoptimize over a saved qk-norm candidate list times each
    candidate's literal plan and, where it exists, its tile-program plan,
    and keeps the fastest; whichever it keeps matches the block-by-block
    emulation of the graph it was given."""
    from tb_numpy import run_graph

    path = os.path.join(GOLDEN, "qknorm_gqa_bs1_subset.json")
    g = MJ.load(path)[10]
    print("case superoptimize qk-norm #10 with its saved list", flush=True)
    opt = g.superoptimize(backend="hip", warmup_iters=2, profile_iters=5, verbose=True, use_graph_dataset=False,
                          use_cached_graphs=False, previous_checkpoint=path)
    log = capsys.readouterr().out
    timed = [l for l in log.splitlines() if l.startswith("[superoptimize hip]")]
    assert any("tb_program" in l for l in timed) and any("tb_program" not in l for l in timed), log
    ins = _inputs(g, (1.0, 0.02, 1.0), seed=10)
    got = opt(inputs=[x.cuda() for x in ins])[0]
    torch.cuda.synchronize()
    ref = run_graph(g, [x.double().numpy() for x in ins])[0]
    err = np.abs(got.float().cpu().numpy() - ref)
    assert not (err > ATOL + RTOL * np.abs(ref)).any(), f"max err {err.max()} (kept {opt._plan.describe()})"


def test_fused_elementwise_bit_identical_to_unfused_steps():
    """Plans whose elementwise trees were fused into single launches
    (yr_hip_graph_ewise) give bit-identical outputs to the same plans run one
    operator per launch, on the saved candidates (every plan that changes)
    and on a broadcasting tree over four inputs in f16 and bf16."""
    import yirage_amd as yr

    checked = 0
    for name, kind, stds in CASES:
        gs = MJ.load(os.path.join(GOLDEN, name))
        seen = set()
        for i, g in enumerate(gs):
            try:
                p1 = g.plan(fuse=True)
                p0 = g.plan(fuse=True, fuse_elementwise=False)
            except YirageHipError:
                continue
            d1 = tuple(p1.describe())
            if d1 == tuple(p0.describe()) or d1 in seen:
                continue
            seen.add(d1)
            print(f"case {name} candidate {i}: {list(d1)}", flush=True)
            dev = [x.cuda() for x in _inputs(g, stds, seed=i)]
            a = g._execute(p0, dev, None)
            b = g._execute(p1, dev, None)
            torch.cuda.synchronize()
            for x, y in zip(a, b):
                assert torch.equal(x, y), f"{name} candidate {i}: fused elementwise differs"
            checked += 1
    for dt in (yr.float16, yr.bfloat16):
        G = yr.new_kernel_graph()
        A = G.new_input(dims=(4, 33, 64), dtype=dt)
        B = G.new_input(dims=(4, 1, 64), dtype=dt)
        C = G.new_input(dims=(1, 33, 1), dtype=dt)
        D = G.new_input(dims=(4, 33, 64), dtype=dt)
        G.mark_output(G.div(G.mul(G.silu(G.add(A, B)), G.exp(C)), G.add(G.square(D), G.exp(G.relu(B)))))
        p1 = G.plan(fuse=True)
        p0 = G.plan(fuse=True, fuse_elementwise=False)
        assert len(p1.describe()) == 1 and p1.describe()[0].startswith("ewise("), p1.describe()
        gen = torch.Generator().manual_seed(7)
        ins = [torch.randn(t.dims, generator=gen).to(dt.torch).cuda() for t in G.inputs]
        a = G._execute(p0, ins, None)[0]
        b = G._execute(p1, ins, None)[0]
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"{dt}: fused elementwise differs"
        x = [t.double() for t in ins]
        ref = (torch.nn.functional.silu(x[0] + x[1]) * torch.exp(x[2])) / (x[3] ** 2 + torch.exp(torch.relu(x[1])))
        err = (b.double() - ref).abs()
        assert (err <= 3e-2 + 3e-2 * ref.abs()).all(), f"{dt}: max err {err.max()}"
        checked += 1
    assert checked >= 4
