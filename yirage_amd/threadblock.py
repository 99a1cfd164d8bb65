"""Threadblock graphs (the body of a kernel graph's `customized` op).

Mirrors python/yirage/threadblock.py of the reference with the shape rules of
src/threadblock/{input_loader,output,forloop_accum,matmul,element_*,
reduction}.cc: an input tile is the device tensor divided along the
input_map dims by the grid and along forloop_dim by forloop_range; an output
multiplies back along output_map / forloop_dim; forloop_accum keeps, reduces
to 1 or to reduction_dimx the last dim.  The hip backend does not generate
per-graph code from a threadblock graph: the kernel-graph planner reads its
outputs as expressions (`expressions()`, and over whole tensors where the
tiling allows), runs the fused kernel of a recognised pattern (RMSNorm +
linear, gated MLP, GQA, linear) and otherwise the generic operators.
"""
from __future__ import annotations

import itertools

from .dtypes import as_dtype

_guid = itertools.count(1)  # shared with kernel.py: device and threadblock tensors never share a guid

# forloop_accum kinds (python/yirage/_cython/core.pyx forloop_accum)
ACCUM_KINDS = {None: "none", "sum": "sum", "mean": "mean", "rms": "rms", "sum_todimx": "sum_todimx"}


class STensor:
    def __init__(self, graph, dims, dt, op, after_accum=False):
        self.graph = graph
        self.dims = tuple(int(d) for d in dims)
        self.dtype = as_dtype(dt)
        self.op = op
        self.after_accum = after_accum
        self.guid = next(_guid)

    @property
    def num_dims(self):
        return len(self.dims)

    def dim(self, i):
        return self.dims[i]

    def __repr__(self):
        return f"STensor{self.dims}"


class TBOp:
    def __init__(self, kind, inputs, **attrs):
        self.kind = kind
        self.inputs = list(inputs)
        self.attrs = attrs
        self.outputs = []


class TBGraph:
    def __init__(self, grid_dim: tuple, block_dim: tuple, forloop_range: int, reduction_dimx: int):
        self.grid_dim = tuple(grid_dim) + (1,) * (3 - len(grid_dim))
        self.block_dim = tuple(block_dim)
        self.forloop_range = int(forloop_range)
        self.reduction_dimx = int(reduction_dimx)
        self.ops: list[TBOp] = []
        self.inputs: list[tuple] = []    # (dtensor, STensor)
        self.outputs: list[tuple] = []   # (STensor, output_map, forloop_dim)
        # the reference python wrapper exposes the graph itself as .cygraph
        self.cygraph = self

    def _op(self, kind, inputs, dims, dt, after_accum=False, **attrs):
        op = TBOp(kind, inputs, **attrs)
        out = STensor(self, dims, dt, op, after_accum)
        op.outputs.append(out)
        self.ops.append(op)
        return out

    def new_input(self, dtensor, input_map: tuple, forloop_dim: int, store_in_dmem: bool = False):
        dims = list(dtensor.dims)
        for g, m in zip(self.grid_dim, tuple(input_map) + (-1,) * (3 - len(input_map))):
            if g > 1 and m >= 0:
                if dims[m] % g:
                    raise ValueError(f"input dim {m} ({dims[m]}) not divisible by grid {g}")
                dims[m] //= g
        if forloop_dim >= 0:
            if dims[forloop_dim] % self.forloop_range:
                raise ValueError(f"forloop dim {forloop_dim} ({dims[forloop_dim]}) not divisible by "
                                 f"forloop_range {self.forloop_range}")
            dims[forloop_dim] //= self.forloop_range
        t = self._op("input", [], dims, dtensor.dtype, dtensor=dtensor, input_map=tuple(input_map),
                     forloop_dim=forloop_dim)
        self.inputs.append((dtensor, t))
        return t

    def new_output(self, stensor: STensor, output_map: tuple, forloop_dim: int = -1, epilogue: str = None):
        self.outputs.append((stensor, tuple(output_map), forloop_dim))

    def output_dims(self, i):
        st, omap, fdim = self.outputs[i]
        dims = list(st.dims)
        for g, m in zip(self.grid_dim, omap + (-1,) * (3 - len(omap))):
            if g > 1 and m >= 0:
                dims[m] *= g
        if fdim >= 0:
            dims[fdim] *= self.forloop_range
        return tuple(dims)

    # ------------------------------------------------------------ ops
    def matmul(self, A: STensor, B: STensor):
        if A.num_dims != B.num_dims or A.dims[-1] != B.dims[-2] or A.dims[:-2] != B.dims[:-2]:
            raise ValueError(f"threadblock matmul shapes {A.dims} x {B.dims}")
        # src/threadblock/matmul.cc:85: the product is after the forloop
        # accumulation when its operands are
        return self._op("matmul", [A, B], A.dims[:-1] + (B.dims[-1],), A.dtype, A.after_accum)

    def _unary(self, kind, A, **attrs):
        return self._op(kind, [A], A.dims, A.dtype, A.after_accum, **attrs)

    def exp(self, A):
        return self._unary("exp", A)

    def silu(self, A):
        return self._unary("silu", A)

    def gelu(self, A):
        return self._unary("gelu", A)

    def relu(self, A):
        return self._unary("relu", A)

    def clamp(self, A, min_val: float, max_val: float):
        return self._unary("clamp", A, min_val=min_val, max_val=max_val)

    def square(self, A):
        return self._unary("square", A)

    def sqrt(self, A):
        return self._unary("sqrt", A)

    def mul_scalar(self, A, scalar: float):
        return self._unary("mul_scalar", A, scalar=scalar)

    def _binary(self, kind, A, B):
        if A.num_dims != B.num_dims or any(a != b and a > 1 and b > 1 for a, b in zip(A.dims, B.dims)):
            raise ValueError(f"threadblock {kind} shapes {A.dims} / {B.dims}")
        return self._op(kind, [A, B], tuple(max(a, b) for a, b in zip(A.dims, B.dims)), A.dtype,
                        A.after_accum or B.after_accum)

    def add(self, A, B):
        return self._binary("add", A, B)

    def mul(self, A, B):
        return self._binary("mul", A, B)

    def div(self, A, B):
        return self._binary("div", A, B)

    def sub(self, A, B):
        return self._binary("sub", A, B)

    def pow(self, A, B):
        return self._binary("pow", A, B)

    def reduction(self, A, dim: int):
        dims = list(A.dims)
        dims[dim] = 1
        return self._op("reduction", [A], dims, A.dtype, A.after_accum, dim=dim)

    def reduction_to_dimx(self, A, dim: int):
        # src/threadblock/reduction.cc:49-58,112: dim `dim` reduced to reduction_dimx
        dims = list(A.dims)
        dims[dim] = self.reduction_dimx
        return self._op("reduction_to_dimx", [A], dims, A.dtype, A.after_accum, dim=dim)

    def reduction_max(self, A, dim: int):
        dims = list(A.dims)
        dims[dim] = 1
        return self._op("reduction_max", [A], dims, A.dtype, A.after_accum, dim=dim)

    def rms_norm(self, A):
        return self._unary("rms_norm", A)

    def concat(self, A, B, dim: int):
        dims = list(A.dims)
        dims[dim] += B.dims[dim]
        return self._op("concat", [A, B], dims, A.dtype, A.after_accum, dim=dim)  # concat.cc:83

    def forloop_accum(self, A: STensor, acc: str = None):
        if acc not in ACCUM_KINDS:
            raise ValueError(f"unknown forloop_accum kind {acc!r}")
        if A.after_accum:
            raise ValueError("forloop_accum of an already accumulated tensor")
        dims = list(A.dims)
        if acc in ("sum", "mean", "rms"):
            dims[-1] = 1
        elif acc == "sum_todimx":
            dims[-1] = self.reduction_dimx
        return self._op("accum", [A], dims, A.dtype, True, acc=ACCUM_KINDS[acc])

    def forloop_accum_rescale(self, A: STensor, B: STensor, acc: str = None):
        dims = list(A.dims)
        if acc == "sum":
            dims[-1] = 1
        return self._op("accum_rescale", [A, B], dims, A.dtype, True, acc=ACCUM_KINDS.get(acc, acc))

    def forloop_accum_max(self, A: STensor):
        return self._op("accum_max", [A], A.dims, A.dtype, True)

    # ------------------------------------------------------------ expressions
    def expressions(self):
        """Each output as a nested tuple over the graph's inputs:
        ('in', i), (kind, *operands) and ('accum', acc, operand)."""
        index = {id(t): i for i, (_, t) in enumerate(self.inputs)}
        memo = {}

        def expr(t: STensor):
            if id(t) in memo:
                return memo[id(t)]
            op = t.op
            if op.kind == "input":
                e = ("in", index[id(t)])
            elif op.kind == "accum":
                e = ("accum", op.attrs["acc"], expr(op.inputs[0]))
            else:
                e = (op.kind,) + tuple(expr(x) for x in op.inputs)
            memo[id(t)] = e
            return e

        return [expr(st) for st, _, _ in self.outputs]


def new_threadblock_graph(grid_dim: tuple, block_dim: tuple, forloop_range: int, reduction_dimx: int) -> TBGraph:
    """python/yirage/__init__.py new_threadblock_graph."""
    return TBGraph(grid_dim, block_dim, forloop_range, reduction_dimx)
