"""A direct numpy emulation of a kernel graph whose customized ops run block
by block and iteration by iteration (test infrastructure).  It follows the
threadblock semantics of the reference's fingerprint executor: tiles are the
device tensor cut along input_map by the grid and along forloop_dim by the
forloop (src/threadblock/input_loader.cc); a forloop accumulator adds its
input over the iterations, `sum` / `sum_todimx` / `rms` / `mean` reducing
the last dim with element j adding j, j + dimx, j + 2 dimx, ...
(include/yirage/threadblock/cuda/reduction.h:41-58, src/threadblock/
graph.cc:460-485, rms as the transpiler lowers it, src/transpiler/
transpile.cc:681-693, mean divided by the count of the summed elements as
include/yirage/threadblock/cuda/forloop_accum.h:89-97 does); a rescale
accumulator multiplies its running value by the rescale tile and adds the
input each iteration, as the transpiler's kernel does
(include/yirage/transpiler/runtime/threadblock/forloop_accum.h:67-93); ops after an accumulator run once after the loop;
outputs are placed by output_map and forloop_dim (output.cc).  float64
throughout.  It is a second, independent reading of the same semantics as
the planner's tile interpreter, which runs every block at once as batched
operators."""
import numpy as np

EPS = 1e-6


def _rms(x):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + EPS)


def _to_dimx(x, axis, to):
    sh = list(x.shape)
    f = sh[axis] // to
    return x.reshape(sh[:axis] + [f, to] + sh[axis + 1:]).sum(axis)


_UN = {"exp": np.exp, "silu": lambda a: a / (1 + np.exp(-a)), "relu": lambda a: np.maximum(a, 0),
       "sqrt": np.sqrt, "square": np.square}
_BIN = {"add": np.add, "mul": np.multiply, "div": np.divide, "pow": np.power, "sub": np.subtract}


def _customized(op, inputs):
    bg = op.attrs["bgraph"]
    R = bg.forloop_range
    grid = bg.grid_dim
    outs = [np.zeros(o.dims) for o in op.outputs]
    for bx in range(grid[0]):
        for by in range(grid[1]):
            for bz in range(grid[2]):
                bc = (bx, by, bz)
                acc = {}
                post = {}
                for it in range(R):
                    v = {}
                    for (dten, st), x in zip(bg.inputs, inputs):
                        sl = [slice(None)] * x.ndim
                        im = tuple(st.op.attrs["input_map"]) + (-1,) * 3
                        start = [0] * x.ndim
                        for a in range(3):
                            if grid[a] > 1 and im[a] >= 0:
                                start[im[a]] += bc[a] * (x.shape[im[a]] // grid[a])
                        fd = st.op.attrs["forloop_dim"]
                        if fd >= 0:
                            start[fd] += it * st.dims[fd]
                        for d in range(x.ndim):
                            sl[d] = slice(start[d], start[d] + st.dims[d])
                        v[id(st)] = x[tuple(sl)]
                    for top in bg.ops:
                        k = top.kind
                        if k == "input" or top.outputs[0].after_accum and k not in ("accum", "accum_max", "accum_rescale"):
                            continue
                        a = [v[id(t)] for t in top.inputs]
                        if k == "accum":
                            x = a[0]
                            if top.attrs["acc"] == "rms":
                                x = x * x
                            acc[id(top)] = acc.get(id(top), 0) + x
                            continue
                        if k == "accum_rescale":  # acc * rescale + input, from zero
                            acc[id(top)] = acc.get(id(top), 0) * a[1] + a[0]
                            continue
                        if k == "accum_max":
                            acc[id(top)] = np.maximum(acc[id(top)], a[0]) if id(top) in acc else a[0]
                            continue
                        v[id(top.outputs[0])] = _eval(k, top, a, bg)
                    for st, omap, ofd in bg.outputs:
                        if ofd >= 0:
                            _place(outs, bg, op, st, omap, ofd, bc, it, v[id(st)])
                # after the loop: accumulator results, then the ops that use them
                for top in bg.ops:
                    if top.kind == "accum_max":
                        post[id(top.outputs[0])] = acc[id(top)]
                    elif top.kind == "accum_rescale":
                        x = acc[id(top)]
                        post[id(top.outputs[0])] = x.sum(-1, keepdims=True) if top.attrs["acc"] == "sum" else x
                    elif top.kind == "accum":
                        x = acc[id(top)]
                        kind = top.attrs["acc"]
                        if kind == "sum":
                            x = x.sum(-1, keepdims=True)
                        elif kind == "sum_todimx":
                            x = _to_dimx(x, x.ndim - 1, bg.reduction_dimx)
                        elif kind == "rms":
                            x = np.sqrt(x.sum(-1, keepdims=True) / (top.inputs[0].dims[-1] * R))
                        elif kind == "mean":
                            x = x.sum(-1, keepdims=True) / (top.inputs[0].dims[-1] * R)
                        elif kind != "none":
                            raise NotImplementedError(kind)
                        post[id(top.outputs[0])] = x
                    elif top.outputs[0].after_accum:
                        post[id(top.outputs[0])] = _eval(top.kind, top, [post[id(t)] for t in top.inputs], bg)
                for st, omap, ofd in bg.outputs:
                    if ofd < 0:
                        _place(outs, bg, op, st, omap, ofd, bc, 0, post[id(st)])
    return outs


def _eval(k, top, a, bg):
    if k in _UN:
        return _UN[k](a[0])
    if k == "mul_scalar":
        return a[0] * top.attrs["scalar"]
    if k == "clamp":
        return np.clip(a[0], top.attrs["min_val"], top.attrs["max_val"])
    if k in _BIN:
        return _BIN[k](a[0], a[1])
    if k == "matmul":
        return a[0] @ a[1]
    if k == "rms_norm":
        return _rms(a[0])
    if k == "reduction":
        return a[0].sum(top.attrs["dim"], keepdims=True)
    if k == "reduction_to_dimx":
        return _to_dimx(a[0], top.attrs["dim"], bg.reduction_dimx)
    if k == "reduction_max":
        return a[0].max(top.attrs["dim"], keepdims=True)
    if k == "concat":
        return np.concatenate(a, top.attrs["dim"])
    raise NotImplementedError(k)


def _place(outs, bg, op, st, omap, ofd, bc, it, tile):
    k = [s for s, _, _ in bg.outputs].index(st)
    out = outs[k]
    om = tuple(omap) + (-1,) * 3
    start = [0] * out.ndim
    for a in range(3):
        if bg.grid_dim[a] > 1 and om[a] >= 0:
            start[om[a]] += bc[a] * (out.shape[om[a]] // bg.grid_dim[a])
    if ofd >= 0:
        start[ofd] += it * st.dims[ofd]
    out[tuple(slice(s, s + d) for s, d in zip(start, st.dims))] = tile


def run_graph(g, inputs):
    """Outputs of kernel graph g (float64) for float64 inputs of its dims."""
    vals = {t.guid: np.asarray(x, np.float64) for t, x in zip(g.inputs, inputs)}
    for op in g.ops:
        a = [vals[t.guid] for t in op.inputs]
        k = op.kind
        if k == "customized":
            for t, o in zip(op.outputs, _customized(op, a)):
                vals[t.guid] = o
            continue
        if k in _UN:
            r = _UN[k](a[0])
        elif k in _BIN:
            r = _BIN[k](a[0], a[1])
        elif k == "matmul":
            r = a[0] @ a[1]
        elif k == "rms_norm":
            r = _rms(a[0])
        elif k == "reduction":
            r = a[0].sum(op.attrs["dim"], keepdims=True)
        else:
            raise NotImplementedError(k)
        vals[op.outputs[0].guid] = r
    return [vals[t.guid] for t, _ in g.outputs]
