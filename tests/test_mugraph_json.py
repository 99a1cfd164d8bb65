"""CPU checks of the muGraph JSON reader / writer (no GPU): the candidate
lists the reference's search saved (tests/golden/saved_mugraphs/, copies of
benchmark/saved_mugraphs/{cuda,mps}/*.json and
tests/ci-tests/qwen2.5/mirage_cached_mugraphs_*.json as shipped) load with
every declared dim agreeing with the shape rules, plan onto the kernels the
reference's search fused them for, and survive a to_json / from_json round
trip with the same structure and plan."""
import json
import os

import pytest

import yirage_amd as yr
from yirage_amd import YirageHipError
from yirage_amd import mugraph_json as MJ

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "saved_mugraphs")

# file -> (number of saved candidates, plan of every candidate or None: none plannable)
EXPECTED = {
    "rmsnorm_bs1.json": (18, ["rmsnorm_linear"]),
    "single_gated_mlp.json": (1, ["gated_mlp"]),
    "single_mqa_bs1.json": (1, ["attention"]),
    "gqa_bs8.json": (10, ["attention"]),
    "mha_bs1.json": (21, None),  # mixed: checked below
    "single_lora.json": (1, ["matmul", "matmul", "matmul", "add"]),
    "ntrans_bs1.json": (9, None),  # mixed: checked below
    "qknorm_gqa_bs1_subset.json": (12, None),  # all run literally: checked below
    "mps_yirage_cached_mugraphs_7310eff92c865e30.json": (21, ["linear"]),
    "mirage_cached_mugraphs_647dd41aeaf656b4.json": (10, ["rmsnorm_linear"]),
    "mirage_cached_mugraphs_64644b2e7bbffb94.json": (14, ["silu", "mul", "linear"]),
}


def _load(name):
    return MJ.load(os.path.join(GOLDEN, name))


def _structure(g):
    """Ops with their kinds, operand positions, output dims and, for
    customized ops, the threadblock graph's output expressions."""
    pos = {t.guid: ("in", i) for i, t in enumerate(g.inputs)}
    out = []
    for k, op in enumerate(g.ops):
        for j, t in enumerate(op.outputs):
            pos[t.guid] = ("op", k, j)
        bg = op.attrs.get("bgraph") if op.kind == "customized" else None
        extra = (tuple(bg.expressions()), bg.grid_dim, bg.block_dim, bg.forloop_range) if bg else None
        out.append((op.kind, tuple(pos[t.guid] for t in op.inputs), tuple(t.dims for t in op.outputs), extra))
    outs = tuple((pos[t.guid], s) for t, s in g.outputs)
    ins = tuple((t.dims, t.strides, t.dtype) for t in g.inputs)
    return ins, tuple(out), outs


@pytest.mark.parametrize("name", sorted(EXPECTED))
def test_saved_candidates_load_and_plan(name):
    n, plan = EXPECTED[name]
    with open(os.path.join(GOLDEN, name)) as f:
        raw = json.load(f)
    gs = _load(name)
    assert len(gs) == len(raw) == n
    for g in gs:
        assert g.outputs, "every saved graph marks an output"
        if plan is not None:
            assert g.plan(fuse=True, fuse_elementwise=False).describe() == plan


def test_mha_candidates_that_plan():
    """Every saved MHA candidate plans: five as the two-op attention form
    (one fused attention step), one as a whole-tensor expression of generic
    steps, and the ones that split the softmax into partial results per
    block run each customized op as one tile program (or, without it,
    literally: tile copies in and out)."""
    gs = _load("mha_bs1.json")
    plans = [g.plan(fuse=True, tb_program=True).describe() for g in gs]
    assert len(plans) == 21
    assert plans.count(["attention"]) == 5
    assert plans.count(["matmul", "exp", "matmul", "reduction", "div"]) == 1
    rest = [p for p in plans if p not in (["attention"], ["matmul", "exp", "matmul", "reduction", "div"])]
    assert len(rest) == 15 and all("tb_program" in p for p in rest)
    lit = [g.plan(fuse=True, tb_program=False).describe() for g in gs]
    assert sum("copy_nd" in p for p in lit) == 15


def test_norm_transformer_candidates_run_as_generic_steps():
    """benchmark/norm_transformer.py's saved candidates: the six whose
    customized op is one whole-tensor expression run as generic rms_norm /
    elementwise steps; the three that divide by an rms accumulator in a
    separate kernel-level div run their customized op as one tile program
    (or literally)."""
    gs = _load("ntrans_bs1.json")
    plans = [g.plan(fuse=True, fuse_elementwise=False, tb_program=True).describe() for g in gs]
    assert plans.count(["rms_norm", "add", "mul", "add", "rms_norm"]) == 6
    assert sum("tb_program" in p for p in plans) == 3
    lit = [g.plan(fuse=True, fuse_elementwise=False, tb_program=False).describe() for g in gs]
    assert sum("copy_nd" in p for p in lit) == 3


def test_grid_placement_must_match_the_cut():
    """A customized op whose output map puts each block's tile where a
    different block's input came from (a block transpose) is not the
    whole-tensor expression its body spells, even with equal dims."""
    def graph(omap):
        g = yr.new_kernel_graph()
        X = g.new_input(dims=(64, 64), dtype=yr.float16)
        tb = yr.new_threadblock_graph(grid_dim=(2, 2, 1), block_dim=(128, 1, 1), forloop_range=1, reduction_dimx=64)
        tX = tb.new_input(dtensor=X, input_map=(0, 1, -1), forloop_dim=-1)
        tb.new_output(stensor=tb.forloop_accum(tb.exp(tX)), output_map=omap)
        O = g.customized([X], tb)[0]
        assert O.dims == (64, 64)
        g.mark_output(O)
        return g
    assert graph((0, 1, -1)).plan(fuse=True).describe() == ["exp"]
    # one tile-program launch instead, or literally: tiles gathered, exp,
    # tiles scattered to the transposed block positions
    assert graph((1, 0, -1)).plan(fuse=True, tb_program=True).describe() == ["tb_program"]
    assert graph((1, 0, -1)).plan(fuse=True, tb_program=False).describe() == ["copy_nd", "exp", "copy_nd"]
    import numpy as np
    from plan_numpy import run_plan

    x = np.random.default_rng(8).normal(0, 1, (64, 64))
    want = np.exp(x).reshape(2, 32, 2, 32).transpose(2, 1, 0, 3).reshape(64, 64)
    for tbp in (True, False):
        got = run_plan(graph((1, 0, -1)).plan(fuse=True, tb_program=tbp), [x])[0]
        assert np.allclose(got, want, rtol=1e-12, atol=0)


def test_unary_chain_tile_program_and_literal_plan():
    """Every unary kind (silu, gelu, relu, clamp, square, sqrt, mul_scalar,
    exp) and add / div in one block-transposed customized op: the tile
    program (numpy VM of its words) and the literal plan against float64
    torch."""
    import numpy as np
    import torch
    from plan_numpy import run_plan

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
    x = np.random.default_rng(9).normal(0, 1, (64, 64))
    xd = torch.tensor(x)
    ref = (torch.nn.functional.silu(xd) + torch.nn.functional.gelu(xd) + torch.relu(xd) + xd.clamp(-0.5, 0.5)
           + xd.abs() + 0.5 * xd) / torch.exp(xd)
    ref = ref.view(2, 32, 2, 32).permute(2, 1, 0, 3).reshape(64, 64).numpy()
    for tbp in (True, False):
        p = g.plan(fuse=True, tb_program=tbp)
        assert ("tb_program" in p.describe()) == tbp
        got = run_plan(p, [x])[0]
        assert np.abs(got - ref).max() <= 1e-12


def _renumber(ops):
    """The JSON text with guids replaced by their order of first use."""
    ids = {}

    def walk(v):
        if isinstance(v, dict):
            return {k: (ids.setdefault(x, len(ids)) if k == "guid" else walk(x)) for k, x in v.items()}
        if isinstance(v, list):
            return [walk(x) for x in v]
        return v
    return json.dumps(walk(ops))


@pytest.mark.parametrize("name", sorted(EXPECTED))
def test_round_trip(name, tmp_path):
    for g in _load(name)[:4]:
        text = json.dumps(MJ.graph_to_json(g))
        g2 = MJ.graph_from_json(json.loads(text))
        assert _structure(g2) == _structure(g)
        assert g2.get_owner_independent_hash() == g.get_owner_independent_hash()
        # what is written is read back to the same text, up to guid numbering
        assert _renumber(MJ.graph_to_json(g2)) == _renumber(json.loads(text))
    g = _load(name)[0]
    path = tmp_path / "g.json"
    g.to_json(str(path))
    h = yr.new_kernel_graph()
    h.from_json(str(path))
    assert _structure(h) == _structure(g)
    assert all(t.graph is h for t in h.inputs)


def test_declared_dims_are_checked(tmp_path):
    with open(os.path.join(GOLDEN, "single_gated_mlp.json")) as f:
        raw = json.load(f)
    mul = [op for op in raw[0] if op["op_type"] == "kn_mul_op"][0]
    mul["output_tensors"][0]["dim"][1] += 8
    with pytest.raises(YirageHipError):
        MJ.graph_from_json(raw[0])


def test_stale_dtype_and_accumulator_names_are_read():
    with open(os.path.join(GOLDEN, "rmsnorm_bs1.json")) as f:
        ops = json.load(f)[0]
    text = json.dumps(ops).replace('"data_type": 940', '"data_type": 921')
    text = text.replace("tb_forloop_accum_", "tb_accum_")
    old = MJ.graph_from_json(json.loads(text))
    new = MJ.graph_from_json(ops)
    assert _structure(old) == _structure(new)


def test_superoptimize_reads_a_previous_checkpoint():
    """The Qwen2 demo's RMSNorm + linear with gamma and a column-major
    weight (demo/qwen2.5/models/modeling_qwen2.py), superoptimized with the
    reference's saved candidate list as previous_checkpoint: the saved
    candidates with this graph's interface are planned too (on CPU the
    first candidate is kept without profiling)."""
    yr.graph_dataset.clear()
    g = yr.new_kernel_graph()
    X = g.new_input(dims=(1, 3584), dtype=yr.float16)
    G = g.new_input(dims=(1, 3584), dtype=yr.float16)
    W = g.new_input(dims=(3584, 37888), strides=(1, 3584), dtype=yr.float16)
    g.mark_output(g.matmul(g.mul(g.rms_norm(X, normalized_shape=(3584,)), G), W))
    ckpt = os.path.join(GOLDEN, "mirage_cached_mugraphs_647dd41aeaf656b4.json")
    opt = g.superoptimize(backend="hip", profile_iters=0, use_graph_dataset=False, previous_checkpoint=ckpt)
    assert opt.backend == "hip" and opt._plan.describe() == ["rmsnorm_linear"]
    # a graph with no kernel of its own: the checkpoint's candidates (same
    # inputs and outputs) are what runs; without them it raises
    h = yr.new_kernel_graph()
    hX = h.new_input(dims=(1, 3584), dtype=yr.float16)
    hG = h.new_input(dims=(1, 3584), dtype=yr.float16)
    hW = h.new_input(dims=(3584, 37888), strides=(1, 3584), dtype=yr.float16)
    # a rescaled accumulator whose rescale tile is not one factor per row
    # (the reference's rescale kernel rejects it too): no fused kernel, no
    # whole-tensor expression and no generic form
    tb = yr.new_threadblock_graph(grid_dim=(592, 1, 1), block_dim=(128, 1, 1), forloop_range=64, reduction_dimx=64)
    tX = tb.new_input(dtensor=hX, input_map=(-1, -1, -1), forloop_dim=1)
    tG = tb.new_input(dtensor=hG, input_map=(-1, -1, -1), forloop_dim=1)
    tW = tb.new_input(dtensor=hW, input_map=(1, -1, -1), forloop_dim=0)
    mm = tb.matmul(tb.mul(tX, tG), tW)
    tb.new_output(stensor=tb.forloop_accum_rescale(mm, tb.exp(tX)), output_map=(1, -1, -1))
    h.mark_output(h.customized([hX, hG, hW], tb)[0])
    with pytest.raises(YirageHipError):
        h.superoptimize(backend="hip", profile_iters=0, use_graph_dataset=False)
    opt = h.superoptimize(backend="hip", profile_iters=0, use_graph_dataset=False, previous_checkpoint=ckpt)
    assert opt._plan.describe() == ["rmsnorm_linear"]
    # the interface differs from every candidate in ckpt: only its own plans
    lora = _load("single_lora.json")[0]
    opt = lora.superoptimize(backend="hip", profile_iters=0, use_graph_dataset=False, previous_checkpoint=ckpt)
    assert opt._plan.describe() == ["matmul", "matmul", "matmul", "add"]


def test_forloop_sum_planned_only_over_the_contraction():
    """A `none` accumulator sums the forloop's tiles: around a matmul whose
    forloop runs over K it is the whole matmul (planned as a linear step);
    when the forloop runs over W's columns instead, the sum is not a matmul
    of the whole tensors (its output is one tile wide) and the graph must
    not be planned as one."""
    def graph(w_forloop_dim, x_forloop_dim):
        g = yr.new_kernel_graph()
        X = g.new_input(dims=(8, 256), dtype=yr.float16)
        W = g.new_input(dims=(256, 256), dtype=yr.float16)
        tb = yr.new_threadblock_graph(grid_dim=(4, 1, 1), block_dim=(128, 1, 1), forloop_range=4, reduction_dimx=64)
        tX = tb.new_input(dtensor=X, input_map=(-1, -1, -1), forloop_dim=x_forloop_dim)
        tW = tb.new_input(dtensor=W, input_map=(1, -1, -1), forloop_dim=w_forloop_dim)
        tb.new_output(stensor=tb.forloop_accum(tb.matmul(tX, tW)), output_map=(1, -1, -1))
        g.mark_output(g.customized([X, W], tb)[0])
        return g
    assert graph(0, 1).plan(fuse=True).describe() == ["linear"]
    # the tile sums run as a tile program instead (or literally)
    assert graph(1, -1).plan(fuse=True, tb_program=True).describe() == ["tb_program"]
    assert "copy_nd" in graph(1, -1).plan(fuse=True, tb_program=False).describe()
    import numpy as np
    from plan_numpy import run_plan
    from tb_numpy import run_graph

    rng = np.random.default_rng(9)
    ins = [rng.normal(0, 1, (8, 256)), rng.normal(0, 1, (256, 256))]
    ref = run_graph(graph(1, -1), ins)[0]
    for tbp in (True, False):
        got = run_plan(graph(1, -1).plan(fuse=True, tb_program=tbp), ins)[0]
        assert np.abs(got - ref).max() <= 1e-9 * max(1.0, np.abs(ref).max())


def test_literal_tile_interpreter_matches_block_emulation():
    """The planner's literal reading of a threadblock graph (block tensors,
    tile gathers and scatters, batched operators; executed here by
    tests/plan_numpy.py) against a block-by-block emulation of the same
    graph (tests/tb_numpy.py), float64, on saved candidates that only the
    literal reading can run; the MHA ones also against softmax(Q K) V."""
    import numpy as np
    import torch
    from plan_numpy import run_plan
    from tb_numpy import run_graph

    rng = np.random.default_rng(0)
    mha = [rng.normal(0, 0.25, (32, 16, 64)), rng.normal(0, 0.25, (32, 64, 4096)), rng.normal(0, 1, (32, 4096, 64))]
    cases = [
        ("ntrans_bs1.json", [rng.normal(0, 1, (8, 4096)) for _ in range(3)], 9),
        ("qknorm_gqa_bs1_subset.json",
         [rng.normal(0, 1, (2, 256, 64)), rng.normal(0, 0.15, (2, 64, 4096)), rng.normal(0, 1, (2, 4096, 64))], 12),
        ("mha_bs1.json", mha, 4),
    ]
    attn = (torch.softmax(torch.tensor(mha[0]) @ torch.tensor(mha[1]), -1) @ torch.tensor(mha[2])).numpy()
    checked = programs = 0
    for name, ins, n in cases:
        for g in _load(name)[:n]:
            try:
                p = g.plan(fuse=True, fuse_elementwise=False, tb_program=False)
            except YirageHipError:
                continue
            if "copy_nd" not in p.describe():
                continue
            got = run_plan(p, ins)[0]
            ref = run_graph(g, ins)[0]
            assert np.abs(got - ref).max() <= 1e-9 * max(1.0, np.abs(ref).max())
            # the same plan with its elementwise trees fused: same values
            pf = g.plan(fuse=True, tb_program=False)
            got_f = run_plan(pf, ins)[0]
            assert np.abs(got_f - got).max() <= 1e-12 * max(1.0, np.abs(got).max())
            if name == "mha_bs1.json":
                assert np.abs(got - attn).max() <= 1e-9
            checked += 1
            # each such customized op as one tile program
            pt = g.plan(fuse=True, tb_program=True)
            if "tb_program" in pt.describe():
                got_t = run_plan(pt, ins)[0]
                assert np.abs(got_t - ref).max() <= 1e-9 * max(1.0, np.abs(ref).max())
                programs += 1
    assert checked >= 3 + 12 + 2
    print("tile programs checked", programs)


def _max_concat_graph():
    """Tiles of X [8, 256] (grid 2 over rows, forloop 4 over columns): the
    running max of exp over the iterations, concatenated with the summed
    per-chunk row maxima."""
    g = yr.new_kernel_graph()
    X = g.new_input(dims=(8, 256), dtype=yr.float16)
    tb = yr.new_threadblock_graph(grid_dim=(2, 1, 1), block_dim=(128, 1, 1), forloop_range=4, reduction_dimx=64)
    tX = tb.new_input(dtensor=X, input_map=(0, -1, -1), forloop_dim=1)
    m = tb.forloop_accum_max(tb.exp(tX))
    s = tb.forloop_accum(tb.reduction_max(tX, 1))
    tb.new_output(stensor=tb.concat(m, s, 1), output_map=(0, -1, -1))
    g.mark_output(g.customized([X], tb)[0])
    return g


def test_literal_max_and_concat():
    import numpy as np
    from plan_numpy import run_plan
    from tb_numpy import run_graph

    g = _max_concat_graph()
    assert "reduction_max" in g.plan(fuse=True, tb_program=False).describe() and g.outputs[0][0].dims == (8, 65)
    assert g.plan(fuse=True, tb_program=True).describe() == ["tb_program"]
    x = np.random.default_rng(1).normal(0, 1, (8, 256))
    ref = run_graph(g, [x])[0]
    for tbp in (True, False):
        got = run_plan(g.plan(fuse=True, tb_program=tbp), [x])[0]
        assert np.abs(got - ref).max() <= 1e-12
    # closed form: max over the row of exp(x) per column position, then the row max sums
    xr = x.reshape(8, 4, 64)
    assert np.allclose(ref[:, :64], np.exp(xr).max(1)) and np.allclose(ref[:, 64], xr.max(2).sum(1))


def _mean_graph():
    """Tiles of X [8, 256] (grid 2 over rows, forloop 4 over columns): the
    mean accumulator of exp over the 256 columns of each row, plus a sum
    accumulator of the same tiles for the ratio check."""
    g = yr.new_kernel_graph()
    X = g.new_input(dims=(8, 256), dtype=yr.float16)
    tb = yr.new_threadblock_graph(grid_dim=(2, 1, 1), block_dim=(128, 1, 1), forloop_range=4, reduction_dimx=64)
    tX = tb.new_input(dtensor=X, input_map=(0, -1, -1), forloop_dim=1)
    e = tb.exp(tX)
    tb.new_output(stensor=tb.forloop_accum(e, "mean"), output_map=(0, -1, -1))
    tb.new_output(stensor=tb.forloop_accum(e, "sum"), output_map=(0, -1, -1))
    outs = g.customized([X], tb)
    g.mark_output(outs[0])
    g.mark_output(outs[1])
    return g


def test_literal_mean_accumulator():
    """The mean forloop accumulator (the fingerprint executor's: the sum over
    the last dim and the iterations over their count) against its closed
    form, the row mean of exp(X), and against sum / 256 of the same tiles;
    also the block-by-block emulation."""
    import numpy as np
    from plan_numpy import run_plan
    from tb_numpy import run_graph

    g = _mean_graph()
    assert g.outputs[0][0].dims == (8, 1)
    x = np.random.default_rng(3).normal(0, 1, (8, 256))
    ref = run_graph(g, [x])
    for tbp in (True, False):
        got = run_plan(g.plan(fuse=True, tb_program=tbp), [x])
        assert np.allclose(got[0][:, 0], np.exp(x).mean(1), rtol=1e-12, atol=0)
        assert np.allclose(got[0], got[1] / 256, rtol=1e-12, atol=0)
        assert np.abs(got[0] - ref[0]).max() <= 1e-12


def _rescale_graph():
    """Tiles of X [8, 256] (grid 2 over rows, forloop 4 over columns): an
    online-softmax style accumulation, acc = acc * exp(-rowmax) + exp(x)
    every iteration, kept whole and with its last dim summed."""
    g = yr.new_kernel_graph()
    X = g.new_input(dims=(8, 256), dtype=yr.float16)
    tb = yr.new_threadblock_graph(grid_dim=(2, 1, 1), block_dim=(128, 1, 1), forloop_range=4, reduction_dimx=64)
    tX = tb.new_input(dtensor=X, input_map=(0, -1, -1), forloop_dim=1)
    s = tb.exp(tb.mul_scalar(tb.reduction_max(tX, 1), -1.0))
    e = tb.exp(tX)
    tb.new_output(stensor=tb.forloop_accum_rescale(e, s), output_map=(0, -1, -1))
    tb.new_output(stensor=tb.forloop_accum_rescale(e, s, "sum"), output_map=(0, -1, -1))
    outs = g.customized([X], tb)
    g.mark_output(outs[0])
    g.mark_output(outs[1])
    return g


def _rescale_closed_form(x):
    """sum_i exp(x_i) prod_{j > i} exp(-max_j) per row, x cut into 4 column
    chunks of 64 (float64)."""
    import numpy as np

    c = x.reshape(8, 4, 64)
    f = np.exp(-c.max(2))  # [8, 4] rescale factor of each iteration
    acc = np.zeros((8, 64))
    for i in range(4):
        acc += np.exp(c[:, i]) * np.prod(f[:, i + 1:], axis=1, keepdims=True)
    return acc, acc.sum(1, keepdims=True)


def test_literal_rescale_accumulator():
    """Rescale accumulators (the transpiler's acc = acc * rescale + input per
    iteration) against the closed form sum_i x_i prod_{j>i} r_j, and against
    the block-by-block emulation."""
    import numpy as np
    from plan_numpy import run_plan
    from tb_numpy import run_graph

    g = _rescale_graph()
    assert [o[0].dims for o in g.outputs] == [(8, 64), (8, 1)]
    x = np.random.default_rng(6).normal(0, 1, (8, 256))
    want, want_sum = _rescale_closed_form(x)
    ref = run_graph(g, [x])
    for tbp in (True, False):
        got = run_plan(g.plan(fuse=True, tb_program=tbp), [x])
        assert np.allclose(got[0], want, rtol=1e-12, atol=0) and np.allclose(got[1], want_sum, rtol=1e-12, atol=0)
        assert np.abs(got[0] - ref[0]).max() <= 1e-12 and np.abs(got[1] - ref[1]).max() <= 1e-12


def test_elementwise_trees_fuse_into_one_launch():
    """Single-consumer trees of elementwise steps become one fused
    elementwise launch (the reference's transpiler fusion rule,
    src/transpiler/resolve_tb_fusion.cc:35-66): the Qwen2 candidate's
    silu * mul, the norm-transformer's add-mul-add; a value read twice or a
    graph output is not folded.  Values (numpy executor, float64) equal the
    unfused plan's."""
    import numpy as np
    from plan_numpy import run_plan

    g = _load("mirage_cached_mugraphs_64644b2e7bbffb94.json")[0]
    assert g.plan(fuse=True).describe() == ["ewise(silu+mul)", "linear"]
    plans = [g.plan(fuse=True).describe() for g in _load("ntrans_bs1.json")]
    assert plans.count(["rms_norm", "ewise(add+mul+add)", "rms_norm"]) == 6
    rng = np.random.default_rng(3)
    for g in _load("ntrans_bs1.json"):
        ins = [rng.normal(0, 1, t.dims) for t in g.inputs]
        a = run_plan(g.plan(fuse=True, fuse_elementwise=False), ins)
        b = run_plan(g.plan(fuse=True), ins)
        for x, y in zip(a, b):
            assert np.abs(x - y).max() <= 1e-12 * max(1.0, np.abs(x).max())
    # a graph-level chain: exp(x) used twice stays materialized
    G = yr.new_kernel_graph()
    X = G.new_input(dims=(16, 64), dtype=yr.float16)
    Y = G.new_input(dims=(16, 1), dtype=yr.float16)
    E = G.exp(X)
    G.mark_output(G.mul(G.add(E, Y), E))
    d = G.plan(fuse=True).describe()
    assert d == ["exp", "ewise(add+mul)"], d


def test_reference_graph_crosses_over_in_mugraph_json(tmp_path):
    """The hip branch of the reference's superoptimize: a graph object that
    only offers the reference's to_json(filename) (here a stand-in writing
    one of the reference's saved files) becomes a graph of this backend,
    with the same interface and plan as loading the file directly."""
    import shutil

    src = os.path.join(GOLDEN, "mirage_cached_mugraphs_647dd41aeaf656b4.json")
    with open(src) as f:
        first = json.dumps(json.load(f)[0])

    class RefGraph:  # the reference's KNGraph surface used by the branch
        def to_json(self, filename):
            with open(filename, "w") as f:
                f.write(first)

    g = yr.from_reference_graph(RefGraph())
    direct = yr.from_reference_graph(first)
    assert g._same_interface(direct)
    assert g.plan(fuse=True).describe() == direct.plan(fuse=True).describe()
    opt = g.superoptimize(backend="hip", profile_iters=0, use_graph_dataset=False)
    assert opt.backend == "hip" and opt._plan.describe() == direct.plan(fuse=True).describe()
    shutil.rmtree(tmp_path, ignore_errors=True)
