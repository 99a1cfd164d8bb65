"""Kernel graphs in the reference's JSON form: the files `KNGraph.to_json` /
`from_json` write and read (one graph: its operator list) and the candidate
lists the reference's search saves and reloads (`previous_checkpoint`,
`benchmark/saved_mugraphs/*.json`: a list of such graphs).

Schema (src/kernel/graph.cc:185-313, src/threadblock/graph.cc:767-951,
include/yirage/kernel/device_tensor.h:139-140, include/yirage/type.h:125-330):
an operator is {op_type, input_tensors, output_tensors, ...}; a device tensor
is {data_type, dim (padded to 4), guid, layout, num_dims}; tensors are
matched by guid.  kn_input_op carries input_strides, kn_output_op
output_strides, kn_customized_op a "bgraph" {grid_dim, block_dim,
forloop_range, reduction_dimx, operators}; tb_input_op carries the device
tensor, input_map and forloop_dim, tb_output_op output_map.  The
threadblock graph's inputs bind to the customized op's inputs in order.

Saved graphs from before the reference renumbered its enums carry data type
921 for fp16 (940 today) and the forloop accumulators as tb_accum_* instead
of tb_forloop_accum_*; both spellings are read, the current ones written.

Every operator is rebuilt through the graph API, so the shape rules apply;
the dims a file declares for each output are then checked against them.
"""
from __future__ import annotations

import json
import os

from . import dtypes
from ._lib import YirageHipError

MAX_DIMS = 4  # yirage::config::MAX_TENSOR_DIMS: dims are written padded to 4
_STALE_DT = {921: 940}

_KN_UNARY = {"kn_exp_op": "exp", "kn_square_op": "square", "kn_sqrt_op": "sqrt", "kn_silu_op": "silu",
             "kn_gelu_op": "gelu", "kn_relu_op": "relu"}
_KN_BINARY = {"kn_add_op": "add", "kn_mul_op": "mul", "kn_div_op": "div", "kn_pow_op": "pow"}
_KN_RED = {"kn_reduction_0_op": 0, "kn_reduction_1_op": 1, "kn_reduction_2_op": 2}

_TB_UNARY = {"tb_exp_op": "exp", "tb_square_op": "square", "tb_sqrt_op": "sqrt", "tb_silu_op": "silu",
             "tb_gelu_op": "gelu", "tb_relu_op": "relu", "tb_rms_norm_op": "rms_norm"}
_TB_BINARY = {"tb_add_op": "add", "tb_mul_op": "mul", "tb_div_op": "div", "tb_sub_op": "sub", "tb_pow_op": "pow"}
_TB_RED = {"tb_reduction_0_op": 0, "tb_reduction_1_op": 1, "tb_reduction_2_op": 2}
_TB_RED_DIMX = {"tb_reduction_0_to_dimx_op": 0, "tb_reduction_1_to_dimx_op": 1, "tb_reduction_2_to_dimx_op": 2}
_TB_RED_MAX = {"tb_reduction_0_max_op": 0, "tb_reduction_1_max_op": 1, "tb_reduction_2_max_op": 2}
_TB_CONCAT = {"tb_concat_0_op": 0, "tb_concat_1_op": 1, "tb_concat_2_op": 2}
# forloop accumulators: kind -> (current name, name in older saved graphs)
_ACC_NAMES = {"none": ("tb_forloop_accum_nored_op", "tb_accum_nored_op"),
              "sum": ("tb_forloop_accum_red_ld_sum_op", "tb_accum_red_ld_sum_op"),
              "mean": ("tb_forloop_accum_red_ld_mean_op", "tb_accum_red_ld_mean_op"),
              "rms": ("tb_forloop_accum_red_ld_rms_op", "tb_accum_red_ld_rms_op"),
              "sum_todimx": ("tb_forloop_accum_redtox_ld_sum_op", "tb_accum_redtox_ld_sum_op")}
_RESCALE_NAMES = {"none": ("tb_forloop_accum_nored_rescale_op", "tb_accum_nored_rescale_op"),
                  "sum": ("tb_forloop_accum_red_ld_sum_rescale_op", "tb_accum_red_ld_sum_rescale_op")}
_MAX_NAMES = ("tb_forloop_accum_max_op", "tb_accum_max_op")
_TB_ACCUM = {n: k for k, names in _ACC_NAMES.items() for n in names}
_TB_RESCALE = {n: k for k, names in _RESCALE_NAMES.items() for n in names}
_API_ACC = {"none": None, "sum": "sum", "mean": "mean", "rms": "rms", "sum_todimx": "sum_todimx"}


def _dtype(code: int):
    code = int(code)
    return dtypes.as_dtype(_STALE_DT.get(code, code))


def _dims(t: dict) -> tuple:
    return tuple(int(d) for d in t["dim"][:int(t["num_dims"])])


def _xyz(m) -> tuple:
    return (int(m["x"]), int(m["y"]), int(m["z"])) if isinstance(m, dict) else tuple(int(v) for v in m)


def _check(what: str, got: tuple, jt: dict):
    want = _dims(jt)
    if tuple(got) != want:
        raise YirageHipError(f"saved graph: {what} has dims {want} in the file, {tuple(got)} by the shape rules")


def _tb_graph(jb: dict, inputs: list):
    from .threadblock import TBGraph

    tb = TBGraph(_xyz(jb["grid_dim"]), _xyz(jb["block_dim"]), int(jb["forloop_range"]), int(jb["reduction_dimx"]))
    st: dict = {}  # file guid -> STensor
    n_in = 0

    def arg(jop, i):
        guid = int(jop["input_tensors"][i]["guid"])
        if guid not in st:
            raise YirageHipError(f"saved graph: threadblock tensor {guid} used before it is defined")
        return st[guid]

    for jop in jb["operators"]:
        kind = jop["op_type"]
        if kind == "tb_input_op":
            if n_in >= len(inputs):
                raise YirageHipError("saved graph: threadblock graph has more inputs than its customized op")
            out = tb.new_input(inputs[n_in], _xyz(jop["input_map"]), int(jop["forloop_dim"]))
            n_in += 1
        elif kind == "tb_output_op":
            # (src/threadblock/graph.cc:797-803: outputs are read back with
            # forloop_dim -1 and no epilogue)
            tb.new_output(arg(jop, 0), _xyz(jop["output_map"]), -1)
            continue
        elif kind == "tb_matmul_op":
            out = tb.matmul(arg(jop, 0), arg(jop, 1))
        elif kind in _TB_UNARY:
            out = getattr(tb, _TB_UNARY[kind])(arg(jop, 0))
        elif kind == "tb_mul_scalar_op":
            if "scalar" not in jop:
                raise YirageHipError("saved graph: tb_mul_scalar_op without its scalar")
            out = tb.mul_scalar(arg(jop, 0), float(jop["scalar"]))
        elif kind == "tb_clamp_op":
            if "min_val" not in jop or "max_val" not in jop:
                raise YirageHipError("saved graph: tb_clamp_op without its bounds")
            out = tb.clamp(arg(jop, 0), float(jop["min_val"]), float(jop["max_val"]))
        elif kind in _TB_BINARY:
            out = getattr(tb, _TB_BINARY[kind])(arg(jop, 0), arg(jop, 1))
        elif kind in _TB_RED:
            out = tb.reduction(arg(jop, 0), _TB_RED[kind])
        elif kind in _TB_RED_DIMX:
            out = tb.reduction_to_dimx(arg(jop, 0), _TB_RED_DIMX[kind])
        elif kind in _TB_RED_MAX:
            out = tb.reduction_max(arg(jop, 0), _TB_RED_MAX[kind])
        elif kind in _TB_CONCAT:
            out = tb.concat(arg(jop, 0), arg(jop, 1), _TB_CONCAT[kind])
        elif kind in _TB_ACCUM:
            out = tb.forloop_accum(arg(jop, 0), _API_ACC[_TB_ACCUM[kind]])
        elif kind in _TB_RESCALE:
            out = tb.forloop_accum_rescale(arg(jop, 0), arg(jop, 1), _API_ACC[_TB_RESCALE[kind]])
        elif kind in _MAX_NAMES:
            out = tb.forloop_accum_max(arg(jop, 0))
        else:
            raise YirageHipError(f"saved graph: threadblock operator {kind!r} is not supported")
        _check(kind, out.dims, jop["output_tensors"][0])
        st[int(jop["output_tensors"][0]["guid"])] = out
    if n_in != len(inputs):
        raise YirageHipError("saved graph: threadblock graph has fewer inputs than its customized op")
    return tb


def graph_from_json(ops: list, graph=None):
    """One kernel graph from its operator list (kernel::Graph from_json)."""
    from .kernel import KNGraph

    g = graph if graph is not None else KNGraph()
    dt: dict = {}  # file guid -> DTensor

    def arg(jop, i):
        guid = int(jop["input_tensors"][i]["guid"])
        if guid not in dt:
            raise YirageHipError(f"saved graph: tensor {guid} used before it is defined")
        return dt[guid]

    for jop in ops:
        kind = jop["op_type"]
        outs = jop.get("output_tensors", [])
        if kind == "kn_input_op":
            t = outs[0]
            strides = jop.get("input_strides")
            res = [g.new_input(_dims(t), tuple(strides) if strides else None, _dtype(t["data_type"]))]
        elif kind == "kn_output_op":
            strides = jop.get("output_strides")
            g.mark_output(arg(jop, 0), tuple(strides) if strides else None)
            continue
        elif kind == "kn_matmul_op":
            res = [g.matmul(arg(jop, 0), arg(jop, 1))]
        elif kind in _KN_UNARY:
            res = [getattr(g, _KN_UNARY[kind])(arg(jop, 0))]
        elif kind == "kn_clamp_op":
            if "min_val" not in jop or "max_val" not in jop:
                raise YirageHipError("saved graph: kn_clamp_op without its bounds")
            res = [g.clamp(arg(jop, 0), float(jop["min_val"]), float(jop["max_val"]))]
        elif kind in _KN_BINARY:
            res = [getattr(g, _KN_BINARY[kind])(arg(jop, 0), arg(jop, 1))]
        elif kind in _KN_RED:
            res = [g.reduction(arg(jop, 0), _KN_RED[kind])]
        elif kind == "kn_rms_norm_op":
            # written by graph_to_json only (the reference reads no rms_norm op)
            if "normalized_shape" not in jop:
                raise YirageHipError("saved graph: kn_rms_norm_op without normalized_shape")
            res = [g.rms_norm(arg(jop, 0), tuple(jop["normalized_shape"]))]
        elif kind == "kn_customized_op":
            ins = [arg(jop, i) for i in range(len(jop["input_tensors"]))]
            res = g.customized(ins, _tb_graph(jop["bgraph"], ins))
        else:
            raise YirageHipError(f"saved graph: operator {kind!r} is not supported")
        if len(res) != len(outs):
            raise YirageHipError(f"saved graph: {kind} has {len(outs)} outputs in the file, {len(res)} built")
        for t, jt in zip(res, outs):
            _check(kind, t.dims, jt)
            dt[int(jt["guid"])] = t
    return g


def load(src):
    """Kernel graphs from a file name, JSON text or parsed JSON: a list of
    graphs (a saved candidate list) or one graph (an operator list)."""
    obj = src
    if isinstance(src, (str, os.PathLike)):
        text = str(src)
        if not text.lstrip().startswith(("[", "{")):
            with open(src) as f:
                text = f.read()
        obj = json.loads(text)
    if not isinstance(obj, list):
        raise YirageHipError("saved graph: expected a JSON list")
    if obj and isinstance(obj[0], list):
        return [graph_from_json(ops) for ops in obj]
    return [graph_from_json(obj)]


# ---------------------------------------------------------------- writing
def _dtensor(t) -> dict:
    dims = list(t.dims) + [0] * (MAX_DIMS - len(t.dims))
    return {"data_type": t.dtype.code, "dim": dims, "guid": t.guid, "layout": "DmemRowMajor",
            "num_dims": len(t.dims)}


def _stensor(t) -> dict:
    dims = list(t.dims) + [0] * (MAX_DIMS - len(t.dims))
    return {"after_accum": bool(t.after_accum), "data_type": t.dtype.code, "dim": dims, "guid": t.guid,
            "layout": "SmemRowMajor", "num_dims": len(t.dims), "smem_offset": 0}


def _xyz_json(v) -> dict:
    v = tuple(v) + (-1,) * (3 - len(v))
    return {"x": v[0], "y": v[1], "z": v[2]}


def _dim3_json(v) -> dict:
    v = tuple(v) + (1,) * (3 - len(v))
    return {"x": v[0], "y": v[1], "z": v[2]}


def _tb_to_json(tb, out_dtensors) -> dict:
    inv_unary = {v: k for k, v in _TB_UNARY.items()}
    inv_binary = {v: k for k, v in _TB_BINARY.items()}
    ops = []
    for op in tb.ops:
        o = op.outputs[0]
        k = op.kind
        j = {"input_tensors": [_stensor(t) for t in op.inputs], "output_tensors": [_stensor(o)]}
        if k == "input":
            j.update(op_type="tb_input_op", dtensor=_dtensor(op.attrs["dtensor"]),
                     input_map=_xyz_json(op.attrs["input_map"]), forloop_dim=op.attrs["forloop_dim"])
        elif k == "matmul":
            j["op_type"] = "tb_matmul_op"
        elif k in inv_unary:
            j["op_type"] = inv_unary[k]
        elif k == "mul_scalar":
            j.update(op_type="tb_mul_scalar_op", scalar=op.attrs["scalar"])
        elif k == "clamp":
            j.update(op_type="tb_clamp_op", min_val=op.attrs["min_val"], max_val=op.attrs["max_val"])
        elif k in inv_binary:
            j["op_type"] = inv_binary[k]
        elif k in ("reduction", "reduction_to_dimx", "reduction_max", "concat"):
            suffix = {"reduction": "", "reduction_to_dimx": "_to_dimx", "reduction_max": "_max"}
            j["op_type"] = (f"tb_concat_{op.attrs['dim']}_op" if k == "concat"
                            else f"tb_reduction_{op.attrs['dim']}{suffix[k]}_op")
        elif k == "accum":
            j["op_type"] = _ACC_NAMES[op.attrs["acc"]][0]
        elif k == "accum_rescale":
            j["op_type"] = _RESCALE_NAMES[op.attrs["acc"] or "none"][0]
        elif k == "accum_max":
            j["op_type"] = _MAX_NAMES[0]
        else:
            raise YirageHipError(f"to_json: threadblock operator {k!r} has no JSON form")
        ops.append(j)
    for (st, omap, _), dtn in zip(tb.outputs, out_dtensors):
        ops.append({"op_type": "tb_output_op", "input_tensors": [_stensor(st)], "output_tensors": [],
                    "dtensor": _dtensor(dtn), "output_map": _xyz_json(omap)})
    return {"grid_dim": _dim3_json(tb.grid_dim), "block_dim": _dim3_json(tb.block_dim),
            "forloop_range": tb.forloop_range, "reduction_dimx": tb.reduction_dimx,
            "graph_level": "thread_block_graph", "smem_offset": 0, "operators": ops}


def graph_to_json(g) -> list:
    """The operator list of kernel graph `g` (kernel::Graph to_json; graph
    inputs first, then operators in creation order, then the outputs)."""
    from .kernel import _row_major

    inv_unary = {v: k for k, v in _KN_UNARY.items()}
    inv_binary = {v: k for k, v in _KN_BINARY.items()}
    ops = []
    for t in g.inputs:
        ops.append({"op_type": "kn_input_op", "input_tensors": [], "output_tensors": [_dtensor(t)],
                    "input_map": _xyz_json(()), "input_strides": list(t.strides)})
    for op in g.ops:
        k = op.kind
        j = {"input_tensors": [_dtensor(t) for t in op.inputs], "output_tensors": [_dtensor(t) for t in op.outputs]}
        if k == "matmul":
            j["op_type"] = "kn_matmul_op"
        elif k in inv_unary:
            j["op_type"] = inv_unary[k]
        elif k == "clamp":
            j.update(op_type="kn_clamp_op", min_val=op.attrs["min_val"], max_val=op.attrs["max_val"])
        elif k in inv_binary:
            j["op_type"] = inv_binary[k]
        elif k == "reduction":
            j["op_type"] = f"kn_reduction_{op.attrs['dim']}_op"
        elif k == "rms_norm":
            j.update(op_type="kn_rms_norm_op", normalized_shape=list(op.attrs["normalized_shape"]))
        elif k == "customized":
            j.update(op_type="kn_customized_op", bgraph=_tb_to_json(op.attrs["bgraph"], op.outputs))
        else:
            raise YirageHipError(f"to_json: operator {k!r} has no JSON form")
        ops.append(j)
    for t, strides in g.outputs:
        ops.append({"op_type": "kn_output_op", "input_tensors": [_dtensor(t)], "output_tensors": [],
                    "output_map": _xyz_json(()),
                    "output_strides": list(strides) if strides is not None else list(_row_major(t.dims))})
    return ops
