"""A numpy executor for the generic steps of a kernel-graph plan (test
infrastructure: it lets CPU tests check what the planner emits -- tile
gathers and scatters, elementwise ops, reductions, matmuls -- against a
float64 restatement of the graph without a GPU).  Values are kept in float64
and not rounded to 16 bits between steps; the plan must use only the
generic operators (no fused kernels)."""
import numpy as np

from yirage_amd import _lib

_UNARY = {
    0: np.exp,
    1: lambda a: a / (1.0 + np.exp(-a)),
    3: lambda a: np.maximum(a, 0.0),
    5: np.sqrt,
    6: np.square,
}


def _f32(bits):
    return float(np.array([bits & 0xFFFFFFFF], np.uint32).view(np.float32)[0])


def _copy_nd(src, p):
    nd = p[0]
    dims, ss, ds = p[2:2 + nd], p[10:10 + nd], p[18:18 + nd]
    idx = np.indices(dims).reshape(nd, -1)
    so = (idx * np.array(ss)[:, None]).sum(0)
    do = (idx * np.array(ds)[:, None]).sum(0)
    return so, do


def run_plan(plan, inputs):
    """inputs: float arrays with each graph input's dims (dense).  Returns
    the graph outputs as float64 arrays of their dims."""
    temps = [np.zeros(int(np.prod(d)), np.float64) for d, _ in plan.temps]
    outs = [np.zeros(int(np.prod(d)), np.float64) for d, _, _ in plan.outputs]
    flat_in = [np.asarray(x, np.float64).reshape(-1) for x in inputs]

    def buf(ref):
        kind, i = ref
        return flat_in[i] if kind == "in" else temps[i] if kind == "tmp" else outs[i]

    for st in plan.steps:
        p = st.params
        src = [buf(r) for r in st.ins]
        dst = buf(st.outs[0])
        k = st.kind
        if k == _lib.OP_COPY_ND:
            so, do = _copy_nd(src[0], p)
            dst[do + p[26]] = src[0][so + (p[27] if len(p) > 27 else 0)]
        elif k == _lib.OP_UNARY:
            n, kind, lo, hi = p[0], p[1], _f32(p[3]), _f32(p[4])
            a = src[0][:n]
            if kind == 7:
                dst[:n] = a * lo
            elif kind == 4:
                dst[:n] = np.clip(a, lo, hi)
            else:
                dst[:n] = _UNARY[kind](a)
        elif k == _lib.OP_BINARY:
            nd, kind = p[0], p[1]
            da, db = p[3:3 + nd], p[3 + nd:3 + 2 * nd]
            a, b = src[0][:int(np.prod(da))].reshape(da), src[1][:int(np.prod(db))].reshape(db)
            r = {0: np.add, 1: np.multiply, 2: np.divide, 3: np.power}[kind](a, b)
            dst[:r.size] = r.reshape(-1)
        elif k == _lib.OP_EWISE:
            nd, nin, npg = p[0], p[1], p[2]
            od = tuple(p[4:4 + nd])
            ind = [tuple(p[4 + nd + i * nd:4 + nd + (i + 1) * nd]) for i in range(nin)]
            prog = p[4 + nd + nin * nd:4 + nd + nin * nd + 5 * npg]
            imm = p[4 + nd + nin * nd + 5 * npg:]
            reg = {}
            last = 0
            for j in range(npg):
                op, d, a, b, kind = prog[5 * j:5 * j + 5]
                if op == 0:
                    v = src[a][:int(np.prod(ind[a]))].reshape(ind[a])
                elif op == 1:
                    x, lo, hi = reg[a], _f32(imm[2 * j]), _f32(imm[2 * j + 1])
                    v = x * lo if kind == 7 else np.clip(x, lo, hi) if kind == 4 else _UNARY[kind](x)
                else:
                    v = {0: np.add, 1: np.multiply, 2: np.divide, 3: np.power}[kind](reg[a], reg[b])
                reg[d] = v
                last = d
            r = np.broadcast_to(reg[last], od)
            dst[:r.size] = r.reshape(-1)
        elif k == _lib.OP_REDUCTION:
            outer, red, inner = p[0], p[1], p[2]
            dst[:outer * inner] = src[0][:outer * red * inner].reshape(outer, red, inner).sum(1).reshape(-1)
        elif k == _lib.OP_REDUCTION_MAX:
            outer, red, inner = p[0], p[1], p[2]
            dst[:outer * inner] = src[0][:outer * red * inner].reshape(outer, red, inner).max(1).reshape(-1)
        elif k == _lib.OP_RMSNORM:
            rows, n, eps = p[0], p[1], _f32(p[3])
            x = src[0][:rows * n].reshape(rows, n)
            dst[:rows * n] = (x / np.sqrt((x * x).mean(1, keepdims=True) + eps)).reshape(-1)
        elif k == _lib.OP_MATMUL:
            batch, m, n, kk = p[0], p[1], p[2], p[3]
            a = src[0][:batch * m * kk].reshape(batch, m, kk)
            b = src[1][:batch * kk * n].reshape(batch, kk, n)
            dst[:batch * m * n] = (a @ b).reshape(-1)
        else:
            raise NotImplementedError(f"step {st.name} (kind {k}) has no numpy form here")
    return [o.reshape(d) for o, (d, _, _) in zip(outs, plan.outputs)]
