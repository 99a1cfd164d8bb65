"""Loading task graphs in the reference's task_graph.json schema
(src/kernel/runtime.cc:847-1318) into a PersistentKernel of the hip backend.

The file lists tasks ({task_type, variant_id, inputs / outputs as {base_ptr,
offset, data_type, dims, strides}, trigger_event, dependent_event, ...}),
not layers.  load_task_graph() groups consecutive tasks of one operator,
recovers the layer each group implements and its operands (tensor names, and
for weights the row pieces each task reads, in output order), and records
the layers on the PersistentKernel, whose compile() then fuses and schedules
them for this backend.  Task types understood:

  101 embedding, 119 rms_norm, 120 linear, 108 linear_with_residual,
  116 paged_attention, 118 silu_mul, 110 / 111 argmax partial / reduce (the
  reference's own tasks, task_register.cc), and this backend's fused
  102 rms_norm_linear (variant 0 plain, 1 + silu_mul, 2 + argmax) and
  1000 prepare_next_batch (graphs written by yr_pk_graph_export_json).

`tensors` binds every base_ptr name to a torch tensor (the reference binds
names to device pointers in construct_task_graph the same way).
"""
from __future__ import annotations

import json

from ._lib import YirageHipError

EMBED, RMSNORM_LINEAR, LINEAR_RES, PAGED_ATTN, SILU_MUL, RMSNORM, LINEAR = 101, 102, 108, 116, 118, 119, 120
ARGMAX_PARTIAL, ARGMAX_REDUCE, PREPARE = 110, 111, 1000
_SKIP = (0, 10)


def _read(graph):
    if isinstance(graph, dict):
        return graph
    text = graph
    if not text.lstrip().startswith("{"):
        with open(graph) as f:
            text = f.read()
    return json.loads(text)


def _group_tasks(tasks):
    """Consecutive tasks of one operator: same type / variant and the same
    operator index (yr.op) when the file carries one, else the same output
    tensor and first input."""
    groups, cur, key = [], [], None
    for t in tasks:
        if t["task_type"] in _SKIP:
            continue
        outs = t.get("outputs", [])
        ins = t.get("inputs", [])
        k = (t["task_type"], t.get("variant_id", 0),
             t["yr"]["op"] if "yr" in t else (outs[0]["base_ptr"] if outs else None,
                                               ins[0]["base_ptr"] if ins else None))
        if k != key and cur:
            groups.append(cur)
            cur = []
        key = k
        cur.append(t)
    if cur:
        groups.append(cur)
    return groups


def _merge(pieces):
    """[(name, row0, rows)] with adjacent contiguous pieces of one tensor merged."""
    out = []
    for n, r0, rows in pieces:
        if out and out[-1][0] == n and out[-1][1] + out[-1][2] == r0:
            out[-1] = (n, out[-1][1], out[-1][2] + rows)
        else:
            out.append((n, r0, rows))
    return out


def _row0(io):
    """First row of a weight piece: byte offset / (row bytes)."""
    esz = 2
    return io["offset"] // (esz * io["strides"][0])


def load_task_graph(graph, pk, tensors: dict, name_prefix: str = "tg"):
    """Record the layers of a task graph on `pk` (a PersistentKernel
    constructed with the graph's meta tensors); call pk.compile() next."""
    g = _read(graph)
    D = {}

    def dt(name):
        if name not in D:
            if name not in tensors:
                raise YirageHipError(f"task graph: tensor '{name}' is not bound")
            D[name] = pk.attach_input(tensors[name], name=name)
        return D[name]

    tmp_n = [0]

    def tmp(like):
        """A placeholder activation between two layers that compile() fuses."""
        from .persistent_kernel import DTensor as PDT
        tmp_n[0] += 1
        return pk._register(PDT(f"{name_prefix}_tmp{tmp_n[0]}", like.dims, like.dtype, None))

    def weight_view(pieces, group=0, ngroups=None):
        pieces = _merge(pieces)
        if len(pieces) == 1 and pieces[0][1] == 0 and pieces[0][2] == tensors[pieces[0][0]].shape[0]:
            return dt(pieces[0][0])
        if ngroups is None:
            # pieces cycling through k source tensors (a shuffle_tensors
            # layout, e.g. [q | k | v] per kv head): one group per cycle
            names = [n for n, _, _ in pieces]
            k = len(dict.fromkeys(names))
            cyc = len(names) % k == 0 and all(names[j] == names[j % k] for j in range(len(names)))
            ngroups = len(names) // k if cyc else 1
        return pk.view_tensor(f"{name_prefix}_w{len(D)}_{len(pk._tensors)}",
                              [(dt(n), r0, rows) for n, r0, rows in pieces], group, ngroups)

    groups = _group_tasks(g["all_tasks"])
    i = 0
    while i < len(groups):
        grp = groups[i]
        t0 = grp[0]
        ty, var = t0["task_type"], t0.get("variant_id", 0)
        ins, outs = t0["inputs"], t0["outputs"]
        if ty == EMBED:
            pk.embed_layer(input=dt(ins[0]["base_ptr"]), weight=dt(ins[1]["base_ptr"]),
                           output=dt(outs[0]["base_ptr"]), grid_dim=(len(grp), 1, 1), block_dim=(128, 1, 1),
                           input_source=1)
        elif ty in (LINEAR, LINEAR_RES, RMSNORM_LINEAR):
            x = dt(ins[0]["base_ptr"])
            out = dt(outs[0]["base_ptr"])
            K = x.dims[1]
            has_norm = ty == RMSNORM_LINEAR
            has_res = ty == LINEAR_RES
            nw = 1 if has_norm else 0
            nr = 1 if has_res else 0

            def wpieces(t):
                return [(p["base_ptr"], _row0(p), p["dims"][0]) for p in t["inputs"][1:len(t["inputs"]) - nw - nr]]
            if var == 1:  # + silu_mul epilogue: each task reads gate rows, then up rows
                grp_rows = t0.get("yr", {}).get("group") or sum(t["outputs"][0]["dims"][1] for t in grp)
                pieces, gate, up, acc = [], [], [], 0
                for t in grp:
                    rows = t["outputs"][0]["dims"][1]
                    ps = wpieces(t)
                    split, run = 0, 0
                    while run < rows:
                        run += ps[split][2]
                        split += 1
                    gate += ps[:split]
                    up += ps[split:]
                    acc += rows
                    if acc % grp_rows == 0:
                        pieces += gate + up
                        gate, up = [], []
                N = acc
                w = weight_view(pieces, grp_rows, N // grp_rows)
            else:
                pieces = [p for t in grp for p in wpieces(t)]
                w = weight_view(pieces)
                N = sum(p[2] for p in pieces)
            norm = dt(ins[-1]["base_ptr"]) if has_norm else None
            res = dt(ins[-1]["base_ptr"]) if has_res else None
            if has_norm:
                xn = tmp(x)
                pk.rmsnorm_layer(input=x, weight=norm, output=xn, grid_dim=(1, 1, 1), block_dim=(128, 1, 1))
                x = xn
            if var == 1:
                from .persistent_kernel import DTensor as PDT
                mid = pk._register(PDT(f"{name_prefix}_mid{i}", (x.dims[0], 2 * N), out.dtype, None))
                pk.linear_layer(input=x, weight=w, output=mid, grid_dim=(len(grp), 1, 1), block_dim=(128, 1, 1))
                pk.silu_mul_layer(input=mid, output=out, grid_dim=(len(grp), 1, 1), block_dim=(128, 1, 1))
            elif res is not None:
                pk.linear_with_residual_layer(input=x, weight=w, residual=res, output=out, grid_dim=(len(grp), 1, 1),
                                              block_dim=(128, 1, 1))
            else:
                pk.linear_layer(input=x, weight=w, output=out, grid_dim=(len(grp), 1, 1), block_dim=(128, 1, 1))
            if var == 2:  # + argmax epilogue: the second output holds the token ids
                tok = dt(outs[1]["base_ptr"])
                pk.argmax_layer(input=out, output=tok, grid_dim=(len(grp), 1, 1), block_dim=(128, 1, 1))
        elif ty == RMSNORM:
            # the reference's separate rms_norm task: its output feeds the next linear
            pk.rmsnorm_layer(input=dt(ins[0]["base_ptr"]), weight=dt(ins[1]["base_ptr"]),
                             output=dt(outs[0]["base_ptr"]), grid_dim=(len(grp), 1, 1), block_dim=(128, 1, 1))
        elif ty == SILU_MUL:
            # each task reads [gate | up] columns of one group: a weight that
            # is already one [gate | up]-shuffled tensor gets that group size
            g_rows = ins[0]["dims"][1] // 2
            prev = pk._layers[-1] if pk._layers else None
            if prev is not None and prev["kind"] == "linear" and not prev["weight"].segments:
                w = prev["weight"]
                prev["weight"] = pk.view_tensor(f"{name_prefix}_gu{i}", [(w, 0, w.dim(0))], g_rows,
                                                w.dim(0) // (2 * g_rows))
            pk.silu_mul_layer(input=dt(ins[0]["base_ptr"]), output=dt(outs[0]["base_ptr"]),
                              grid_dim=(len(grp), 1, 1), block_dim=(128, 1, 1))
        elif ty == PAGED_ATTN:
            # operands: input, k_cache, v_cache, [q_norm, k_norm (1-D)], [cos, sin]
            names = [p["base_ptr"] for p in ins]
            rest = names[3:]
            qn = kn = None
            if len(rest) >= 2 and len(ins[3]["dims"]) == 1 and len(ins[4]["dims"]) == 1:
                qn, kn = dt(rest[0]), dt(rest[1])
                rest = rest[2:]
            cos = dt(rest[0]) if len(rest) > 0 else None
            sin = dt(rest[1]) if len(rest) > 1 else None
            pk.paged_attention_layer(input=dt(names[0]), k_cache=dt(names[1]), v_cache=dt(names[2]), q_norm=qn,
                                     k_norm=kn, cos_pos_embed=cos, sin_pos_embed=sin,
                                     output=dt(outs[0]["base_ptr"]), grid_dim=(len(grp), 1, 1), block_dim=(128, 1, 1))
        elif ty == ARGMAX_PARTIAL:
            nxt = groups[i + 1] if i + 1 < len(groups) else None
            if not nxt or nxt[0]["task_type"] != ARGMAX_REDUCE:
                raise YirageHipError("task graph: argmax_partial without argmax_reduce")
            pk.argmax_layer(input=dt(ins[0]["base_ptr"]), output=dt(nxt[0]["outputs"][0]["base_ptr"]),
                            grid_dim=(len(grp), 1, 1), block_dim=(128, 1, 1))
            i += 1
        elif ty == PREPARE:
            pk.prepare_batch_layer()
        else:
            raise YirageHipError(f"task graph: task type {ty} is not supported by the hip backend")
        i += 1
    return pk
