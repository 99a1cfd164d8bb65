"""A numpy executor for the generic steps of a kernel-graph plan (test
infrastructure: it lets CPU tests check what the planner emits -- tile
gathers and scatters, elementwise ops, reductions, matmuls -- against a
float64 restatement of the graph without a GPU).  Values are kept in float64
and not rounded to 16 bits between steps; the plan must use only the
generic operators and tile programs (no fused kernels)."""
import numpy as np

from yirage_amd import _lib

from scipy.special import erf as _erf

_UNARY = {
    0: np.exp,
    1: lambda a: a / (1.0 + np.exp(-a)),
    2: lambda a: 0.5 * a * (1.0 + _erf(a / np.sqrt(2.0))),
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


def _tb_program(words, srcs, dsts):
    """The tile program of a customized op (yr_hip_tb_program's word format,
    yirage_amd/csrc/tb_program.hip), block by block and iteration by
    iteration, float64, no rounding: a third reading of the threadblock
    semantics, checked against tests/tb_numpy.py and on the GPU against the
    kernel.  The LDS is emulated at its byte offsets (one slot per 16 bits,
    a wide tile's second slot holding a guard), so tiles the program lets
    share space while both are live corrupt the values (or trip the guard)."""
    w = list(words)
    R, nt, ni, no, nout, lds_bytes, dimx, gx, gy, gz = w[2], w[3], w[4], w[5], w[6], w[7], w[8], w[9], w[10], w[11]
    pos = 12
    tiles = []  # (halfword offset, dims, wide)
    for _ in range(nt):
        off, nd = w[pos], w[pos + 1]
        tiles.append((off // 2, tuple(w[pos + 2:pos + 2 + nd]), w[pos + 6]))
        pos += 7
    ins = [w[pos + 10 * i:pos + 10 * (i + 1)] for i in range(ni)]
    pos += 10 * ni
    ops = [w[pos + 9 * i:pos + 9 * (i + 1)] for i in range(no)]
    pos += 9 * no
    outs = [w[pos + 11 * i:pos + 11 * (i + 1)] for i in range(nout)]
    grid = (gx, gy, gz)
    GUARD = -7.25e300
    mem = np.full(lds_bytes // 2 + 2, np.nan)

    def get(i):
        h, dims, wide = tiles[i]
        n = int(np.prod(dims))
        if wide:
            assert (mem[h + 1:h + 2 * n:2] == GUARD).all(), f"wide tile {i} overwritten while live"
            return mem[h:h + 2 * n:2].reshape(dims).copy()
        return mem[h:h + n].reshape(dims).copy()

    def put(i, v):
        h, dims, wide = tiles[i]
        n = int(np.prod(dims))
        v = np.broadcast_to(v, dims).reshape(-1)
        if wide:
            mem[h:h + 2 * n:2] = v
            mem[h + 1:h + 2 * n:2] = GUARD
        else:
            mem[h:h + n] = v

    def sl(rec, it, b):
        dims = tiles[rec[0]][1]
        gd = rec[2:2 + len(dims)]
        start = [0] * len(dims)
        for a in range(3):
            m = rec[6 + a]
            if m >= 0:
                start[m] += b[a] * (gd[m] // grid[a])
        if rec[9] >= 0:
            start[rec[9]] += it * dims[rec[9]]
        return gd, tuple(slice(s, s + d) for s, d in zip(start, dims))

    def run(o):
        kind, out, a = o[0], o[1], get(o[2])
        if kind == 1:
            lo, hi = _f32(o[5]), _f32(o[6])
            r = a * lo if o[4] == 7 else np.clip(a, lo, hi) if o[4] == 4 else _UNARY[o[4]](a)
        elif kind == 2:
            r = {0: np.add, 1: np.multiply, 2: np.divide, 3: np.power, 4: np.subtract}[o[4]](a, get(o[3]))
        elif kind == 3:
            r = a @ get(o[3])
        elif kind in (4, 5):
            dim, to = o[4], (o[5] if kind == 4 else 1)
            sh = a.shape
            x = a.reshape(sh[:dim] + (sh[dim] // to, to) + sh[dim + 1:])
            r = x.sum(dim) if kind == 4 else x.max(dim)
        elif kind == 6:
            r = a / np.sqrt((a * a).mean(-1, keepdims=True) + _f32(o[5]))
        elif kind == 7:
            r = np.concatenate([a, get(o[3])], o[4])
        else:
            raise NotImplementedError(kind)
        put(out, r.reshape(tiles[out][1]))

    for b in np.ndindex(gx, gy, gz):
        mem[:] = np.nan
        for it in range(R):
            for rec in ins:
                if it == 0 or rec[9] >= 0:
                    gd, s = sl(rec, it, b)
                    put(rec[0], srcs[rec[1]].reshape(gd)[s])
            if it == 0:
                for o in ops:
                    if o[0] == 8:
                        put(o[8], np.full(tiles[o[8]][1], -np.inf if o[4] == 5 else 0.0))
            for o in ops:
                if o[7]:
                    continue
                if o[0] == 8:
                    acc, x = get(o[8]), get(o[2])
                    if o[4] in (6, 7):
                        acc = acc * get(o[3]) + x
                    elif o[4] == 5:
                        acc = np.maximum(acc, x)
                    else:
                        acc = acc + (x * x if o[4] == 3 else x)
                    put(o[8], acc)
                else:
                    run(o)
            for rec in outs:
                if rec[9] >= 0 and rec[10] == 0:
                    gd, s = sl(rec, it, b)
                    dsts[rec[1]].reshape(gd)[s] = get(rec[0])
        for o in ops:
            if o[0] != 8:
                continue
            acc, kind = get(o[8]), o[4]
            n = acc.shape[-1]
            if kind in (0, 5, 6):
                r = acc
            elif kind == 2:
                r = acc.reshape(acc.shape[:-1] + (n // dimx, dimx)).sum(-2)
            else:
                r = acc.sum(-1, keepdims=True)
                if kind == 4:
                    r = r / (n * R)
                elif kind == 3:
                    r = np.sqrt(r / (n * R))
            put(o[1], r.reshape(tiles[o[1]][1]))
        for o in ops:
            if o[7] and o[0] != 8:
                run(o)
        for rec in outs:
            if rec[9] >= 0 and rec[10] == 0:
                continue
            for it in range(R if rec[9] >= 0 else 1):
                gd, s = sl(rec, it, b)
                dsts[rec[1]].reshape(gd)[s] = get(rec[0])


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
        if k == _lib.OP_TB_PROGRAM:
            _tb_program(p[4:], src, [buf(r) for r in st.outs])
        elif k == _lib.OP_COPY_ND:
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
