"""PersistentKernel for the `hip` backend.

Mirrors python/yirage/persistent_kernel.py:217-1347 of the reference: the
same constructor arguments and meta tensors, attach_input / new_tensor /
fuse_tensors / shuffle_tensors, the *_layer builders, compile() and
__call__().  compile() runs a fusion pass over the recorded layers
(rmsnorm -> linear becomes one rmsnorm_linear task; a [gate | up] linear
followed by silu_mul becomes one task with a SiLU-mul epilogue; the LM-head
linear followed by argmax_partial / argmax_reduce becomes one task with an
argmax epilogue), serialises the op list to JSON and hands it to the C++
task-graph builder in libyirage_hip.so, which emits per-worker queues and
events for the gfx950 megakernel.  No code is generated or compiled at run
time.
"""
from __future__ import annotations

import ctypes
import json
import math
from dataclasses import dataclass, field

import torch

from . import _lib
from ._lib import YirageHipError, check, lib

valid_persistent_kernel_modes = {"offline", "online", "onepass"}

# dtype tags (include/yirage/type.h:84-120 values)
float16, bfloat16, float32, int32, int64 = (_lib.DTYPE_F16, _lib.DTYPE_BF16, _lib.DTYPE_F32, _lib.DTYPE_I32,
                                            _lib.DTYPE_I64)
_TORCH2DT = {torch.float16: float16, torch.bfloat16: bfloat16, torch.float32: float32, torch.int32: int32,
             torch.int64: int64}
_DT2TORCH = {v: k for k, v in _TORCH2DT.items()}


@dataclass(eq=False)
class DTensor:
    """A kernel-graph tensor: a name, a shape and (once bound) device memory.
    Shuffled / fused tensors are views over row segments of their sources."""
    name: str
    dims: tuple
    dtype: int
    tensor: torch.Tensor | None = None
    segments: list = field(default_factory=list)   # [(DTensor, row0, rows)] for views
    group: int = 0                                  # rows per source chunk of a shuffle
    ngroups: int = 1                                # number of shuffle groups
    ll: bool = False                                # stored as tagged words (see _link_tensors)

    @property
    def num_dims(self) -> int:
        return len(self.dims)

    def dim(self, i: int) -> int:
        return self.dims[i]


def get_configurations_from_gpu(rank: int = 0):
    """(num_workers, num_schedulers).  One worker per CU; the hip backend has
    no scheduler workgroups (python/yirage/utils.py:31-57 sizes both for
    NVIDIA parts)."""
    props = torch.cuda.get_device_properties(rank)
    return props.multi_processor_count, 0


class PersistentKernel:
    # attention tasks take about 1 / ATTN_SPLIT_DIVISOR of the workers
    ATTN_SPLIT_DIVISOR = 2

    def __init__(self, mode: str, world_size: int, mpi_rank: int, num_workers: int, num_local_schedulers: int,
                 num_remote_schedulers: int, max_seq_length: int, max_num_batched_requests: int,
                 max_num_batched_tokens: int, max_num_pages: int, page_size: int, eos_token_id: int,
                 meta_tensors: dict, profiler_tensor: torch.Tensor | None = None, trace_name: str = "",
                 spec_decode_config=None, use_cutlass_kernel: bool = False):
        if mode not in valid_persistent_kernel_modes:
            raise ValueError(f"Invalid persistent kernel mode: {mode}")
        if world_size != 1:
            raise YirageHipError("hip backend: the persistent kernel runs on one GPU (world_size must be 1)")
        if spec_decode_config is not None:
            raise YirageHipError("hip backend: speculative decoding is not supported")
        if max_num_batched_tokens > 16:
            raise YirageHipError("hip backend: max_num_batched_tokens must be <= 16")
        self.mode = mode
        self.world_size = world_size
        self.mpi_rank = mpi_rank
        self.num_workers = num_workers
        self.num_local_schedulers = num_local_schedulers
        self.num_remote_schedulers = num_remote_schedulers
        self.max_seq_length = max_seq_length
        self.max_num_batched_requests = max_num_batched_requests
        self.max_num_batched_tokens = max_num_batched_tokens
        self.max_num_pages = max_num_pages
        self.page_size = page_size
        self.eos_token_id = eos_token_id
        self.meta_tensors = meta_tensors
        self.profiler_tensor = profiler_tensor
        self.trace_name = trace_name
        self.total_num_requests = meta_tensors["tokens"].shape[0]
        assert self.max_seq_length == meta_tensors["tokens"].shape[1]
        assert meta_tensors["qo_indptr_buffer"].shape == (max_num_batched_requests + 1,)
        assert meta_tensors["paged_kv_indptr_buffer"].shape == (max_num_batched_requests + 1,)
        assert meta_tensors["paged_kv_indices_buffer"].shape == (max_num_pages,)
        assert meta_tensors["paged_kv_last_page_len_buffer"].shape == (max_num_batched_requests,)
        # element types of the meta tensors (persistent_kernel.py:268-279 of the reference)
        want = {"step": torch.int32, "tokens": torch.int64, "input_tokens": torch.int64,
                "output_tokens": torch.int64, "num_new_tokens": torch.int32, "prompt_lengths": torch.int32,
                "qo_indptr_buffer": torch.int32, "paged_kv_indptr_buffer": torch.int32,
                "paged_kv_indices_buffer": torch.int32, "paged_kv_last_page_len_buffer": torch.int32}
        for key, dt in want.items():
            t = meta_tensors.get(key)
            if t is not None and t.dtype != dt:
                raise YirageHipError(f"meta tensor {key} must be {dt}, got {t.dtype}")
        self._tensors: dict[str, DTensor] = {}
        self._layers: list[dict] = []
        self._owned: list[torch.Tensor] = []
        self._graph = None
        self._handle = None
        self._is_compiled = False
        self.__finalized__ = False
        self.ops: list[dict] = []

    # ------------------------------------------------------------ tensors
    def _register(self, t: DTensor) -> DTensor:
        if t.name in self._tensors:
            raise YirageHipError(f"duplicate tensor name {t.name}")
        self._tensors[t.name] = t
        return t

    def attach_input(self, torch_tensor: torch.Tensor, name: str = None) -> DTensor:
        assert name is not None
        dims = tuple(torch_tensor.shape)
        strides = torch_tensor.stride()
        for d in range(len(dims) - 1):
            assert strides[d] == strides[d + 1] * dims[d + 1], "row-major tensors only"
        if torch_tensor.dtype not in _TORCH2DT:
            raise YirageHipError(f"unsupported dtype {torch_tensor.dtype}")
        return self._register(DTensor(name, dims, _TORCH2DT[torch_tensor.dtype], torch_tensor))

    def new_tensor(self, dims: tuple, strides: tuple = None, dtype: int = bfloat16, name: str = None,
                   io_category: str = "cuda_tensor") -> DTensor:
        assert name is not None
        if io_category not in ("cuda_tensor", "nvshmem_tensor"):
            raise RuntimeError(f"Invalid io_category: {io_category}")
        dtype = int(dtype)  # a yirage_amd dtype (yr.bfloat16) or its integer code
        t = torch.zeros(dims, dtype=_DT2TORCH[dtype], device=self.meta_tensors["qo_indptr_buffer"].device)
        self._owned.append(t)
        return self._register(DTensor(name, tuple(dims), dtype, t))

    def _view(self, inputs, num_groups: int, name: str, shuffled: bool) -> DTensor:
        rows = [t.dim(0) for t in inputs]
        for t in inputs:
            assert t.num_dims == 2 and t.dim(1) == inputs[0].dim(1)
            assert t.dim(0) % num_groups == 0
        segs = []
        if shuffled:
            # group g: rows g*r_i/num_groups .. of every input in turn (runtime.cc:804-842)
            for g in range(num_groups):
                for t, r in zip(inputs, rows):
                    c = r // num_groups
                    segs.append((t, g * c, c))
        else:
            for t, r in zip(inputs, rows):
                segs.append((t, 0, r))
        v = DTensor(name, (sum(rows), inputs[0].dim(1)), inputs[0].dtype, None, segs, rows[0] // num_groups,
                    num_groups if shuffled else 1)
        return self._register(v)

    def view_tensor(self, name: str, segments: list, group: int = 0, ngroups: int = 1) -> DTensor:
        """A weight made of row pieces [(DTensor, row0, rows), ...] in order
        (what fuse_tensors / shuffle_tensors produce), e.g. when a task graph
        file lists the pieces each task reads."""
        src = segments[0][0]
        for t, r0, n in segments:
            assert t.num_dims == 2 and t.dim(1) == src.dim(1) and 0 <= r0 and r0 + n <= t.dim(0)
        rows = sum(n for _, _, n in segments)
        return self._register(DTensor(name, (rows, src.dim(1)), src.dtype, None, list(segments), group, ngroups))

    def fuse_tensors(self, inputs: list, fused_dim: int, num_groups: int, name: str = None) -> DTensor:
        assert fused_dim == 0
        return self._view(inputs, num_groups, name, shuffled=False)

    def shuffle_tensors(self, inputs: list, shuffled_dim: int, num_groups: int, name: str = None) -> DTensor:
        assert shuffled_dim == 0
        return self._view(inputs, num_groups, name, shuffled=True)

    # ------------------------------------------------------------ layers
    def _add(self, kind, **kw):
        self._layers.append(dict(kind=kind, **kw))

    def embed_layer(self, input: DTensor, weight: DTensor, output: DTensor, grid_dim: tuple, block_dim: tuple,
                    input_source: int = 0):
        self._add("embed", input=input, weight=weight, output=output)

    def rmsnorm_layer(self, input: DTensor, weight: DTensor, output: DTensor, grid_dim: tuple, block_dim: tuple):
        assert input.num_dims == 2 and output.num_dims == 2
        self._add("rmsnorm", input=input, weight=weight, output=output)

    def rmsnorm_linear_layer(self, input: DTensor, weight_norm: DTensor, weight_linear: DTensor, output: DTensor,
                             grid_dim: tuple, block_dim: tuple):
        self._add("rmsnorm_linear", input=input, norm=weight_norm, weight=weight_linear, output=output)

    def linear_layer(self, input: DTensor, weight: DTensor, output: DTensor, grid_dim: tuple, block_dim: tuple):
        self._add("linear", input=input, weight=weight, output=output, residual=None)

    def linear_with_residual_layer(self, input: DTensor, weight: DTensor, residual: DTensor, output: DTensor,
                                   grid_dim: tuple, block_dim: tuple):
        self._add("linear", input=input, weight=weight, output=output, residual=residual)

    def silu_mul_layer(self, input: DTensor, output: DTensor, grid_dim: tuple, block_dim: tuple):
        self._add("silu_mul", input=input, output=output)

    def paged_attention_layer(self, input: DTensor, k_cache: DTensor, v_cache: DTensor, q_norm: DTensor,
                              k_norm: DTensor, cos_pos_embed: DTensor, sin_pos_embed: DTensor, output: DTensor,
                              grid_dim: tuple, block_dim: tuple):
        """python/yirage/persistent_kernel.py:532-609: RoPE (cos / sin
        [seq, head_dim]) and, with q_norm / k_norm ([head_dim] each, both or
        neither), per-head RMSNorm of q and the new k before it (eps 1e-6)."""
        assert k_cache.dim(0) == self.max_num_pages and k_cache.dim(1) == self.page_size
        head_dim = k_cache.dim(3)
        if (q_norm is None) != (k_norm is None):
            raise YirageHipError("paged_attention_layer: q_norm and k_norm come together")
        if q_norm is not None:
            for w in (q_norm, k_norm):
                if w.num_dims != 1 or w.dim(0) != head_dim:
                    raise YirageHipError("paged_attention_layer: q_norm / k_norm must be [head_dim]")
        self._add("attention", input=input, k_cache=k_cache, v_cache=v_cache, cos=cos_pos_embed,
                  sin=sin_pos_embed, q_norm=q_norm, k_norm=k_norm, output=output,
                  num_q_heads=output.dim(1) // head_dim, num_kv_heads=k_cache.dim(2), head_dim=head_dim)

    def argmax_partial_layer(self, input: DTensor, output: tuple, grid_dim: tuple, block_dim: tuple):
        self._add("argmax_partial", input=input, output=output)

    def argmax_reduce_layer(self, input: tuple, output: DTensor, grid_dim: tuple, block_dim: tuple):
        self._add("argmax_reduce", input=input, output=output)

    def argmax_layer(self, input: DTensor, output: DTensor, grid_dim: tuple, block_dim: tuple):
        self._add("argmax_partial", input=input, output=None)
        self._add("argmax_reduce", input=None, output=output)

    def prepare_batch_layer(self):
        """The on-device batch/page manager (prepare_next_batch of
        persistent_kernel.cuh:169-322; in mode="online", the single-request
        step advance of :325-351).  It must be the last layer recorded:
        every attention task reads the batch metadata once at launch start,
        and prepare_batch rewrites it for the next launch (compile() refuses
        any other placement)."""
        self._add("prepare_batch")

    # ------------------------------------------------------------ fusion + JSON
    def _segments(self, w: DTensor):
        return [(s.name, r0, n) for (s, r0, n) in w.segments] if w.segments else [(w.name, 0, w.dim(0))]

    @staticmethod
    def _rows_per_task(n_rows: int, num_workers: int, gran: int, max_rows: int | None = None) -> int:
        """Even rows per task dividing `gran`, minimising the per-worker
        makespan ceil(tasks / workers) * (rows + 8): a task costs about
        eight rows of streaming in fixed work (ties -> fewer tasks)."""
        best = None
        cands = [r for r in range(2, gran + 1, 2) if gran % r == 0] if gran else \
            list(range(2, n_rows + 2, 2))
        for r in cands:
            if max_rows and r > max_rows:
                continue
            tasks = -(-n_rows // r)
            span = -(-tasks // num_workers) * (r + 8)
            key = (span, tasks)
            if best is None or key < best[0]:
                best = (key, r)
        if best is None:
            raise YirageHipError(f"no valid rows-per-task for {n_rows} rows (granularity {gran})")
        return best[1]

    def _fuse(self):
        L = self._layers
        for i, l in enumerate(L):
            if l["kind"] == "prepare_batch" and i != len(L) - 1:
                raise YirageHipError("hip backend: prepare_batch_layer must be the last layer of the graph "
                                     "(attention reads the batch metadata at launch start)")
        consumers = {}
        for i, l in enumerate(L):
            for k in ("input", "norm", "residual"):
                v = l.get(k)
                if isinstance(v, DTensor):
                    consumers.setdefault(v.name, []).append(i)
        ops = []
        i = 0
        W = self.num_workers
        attn_free = {}  # attention output -> workers its mergers occupy (left free by the next linear op)
        while i < len(L):
            l = L[i]
            k = l["kind"]
            nxt = L[i + 1] if i + 1 < len(L) else None
            if k == "embed":
                ops.append(dict(type="embed", tokens=l["input"].name, table=l["weight"].name,
                                out=l["output"].name, tasks=max(1, l["weight"].dim(1) // 512)))
                i += 1
                continue
            if k == "rmsnorm":
                if not (nxt and nxt["kind"] == "linear" and nxt["input"] is l["output"] and nxt["residual"] is None):
                    raise YirageHipError("hip backend: rmsnorm_layer must feed a linear_layer (fused into one task)")
                l = dict(kind="rmsnorm_linear", input=l["input"], norm=l["weight"], weight=nxt["weight"],
                         output=nxt["output"])
                i += 1
                nxt = L[i + 1] if i + 1 < len(L) else None
                k = "rmsnorm_linear"
            if k in ("rmsnorm_linear", "linear"):
                w = l["weight"]
                # a linear op right after an attention op with merger splits
                # leaves the mergers' workers free: they finish the attention
                # last, and a task there would start its weight stream late
                Wl = W - attn_free.get(l["input"].name, 0)
                K = w.dim(1)
                op = dict(x=l["input"].name, weight=self._segments(w), out=l["output"].name)
                if k == "rmsnorm_linear":
                    op.update(type="rmsnorm_linear", norm=l["norm"].name, eps=1e-6)
                else:
                    op.update(type="linear")
                    if l.get("residual") is not None:
                        op["residual"] = l["residual"].name
                seg_rows = [n for (_, _, n) in op["weight"]]
                # a task may straddle one weight-segment boundary: rows per task
                # <= the smallest segment and dividing the shuffle group (so no
                # task crosses a kv-head group of a QKV projection)
                if w.segments:
                    gran = w.dim(0) // w.ngroups
                    max_seg = min(seg_rows)
                else:
                    gran, max_seg = 0, None
                tm8 = self.max_num_batched_tokens > 1
                max_rows = 16 if (tm8 and K > 4096) else None
                if self.max_num_batched_tokens > 8 and max_rows is None:
                    # 16-token tiles: a task's partial-sum slots hold (16-row
                    # tiles + 7) x 16 x 16 floats of 8192 (400 rows; 192 rows
                    # of [gate | up] pairs)
                    max_rows = 192 if nxt and nxt["kind"] == "silu_mul" else 400
                if nxt and nxt["kind"] == "silu_mul" and nxt["input"] is l["output"]:
                    two_src = w.segments and len(set(s.name for s, _, _ in w.segments)) == 2
                    one_shuffled = w.segments and len(w.segments) == 1 and w.group > 0  # pre-shuffled [gate | up]
                    if k != "rmsnorm_linear" or not (two_src or one_shuffled):
                        raise YirageHipError("hip backend: silu_mul must follow an rmsnorm+linear over shuffled "
                                             "[gate, up] weights")
                    op["type"] = "rmsnorm_linear_silu"
                    op["group"] = w.group
                    op["out"] = nxt["output"].name
                    op["rows_per_task"] = self._rows_per_task(w.dim(0) // 2, W, w.group, max_rows)
                    i += 2
                elif nxt and nxt["kind"] == "argmax_partial" and nxt["input"] is l["output"]:
                    red = L[i + 2] if i + 2 < len(L) else None
                    if not red or red["kind"] != "argmax_reduce":
                        raise YirageHipError("argmax_partial_layer must be followed by argmax_reduce_layer")
                    if k != "rmsnorm_linear":
                        raise YirageHipError("hip backend: argmax must follow the final rmsnorm+linear")
                    op["type"] = "rmsnorm_linear_argmax"
                    op["tokens_out"] = red["output"].name
                    op["vocab"] = int(getattr(self, "vocab_size", None) or w.dim(0))
                    op["rows_per_task"] = self._rows_per_task(w.dim(0), W, 0, max_rows)
                    i += 3
                else:
                    lim = min(x for x in (max_rows, max_seg) if x) if (max_rows or max_seg) else None
                    op["rows_per_task"] = self._rows_per_task(w.dim(0), Wl, gran, lim)
                    i += 1
                ops.append(op)
                continue
            if k == "attention":
                per = self.max_num_batched_requests * l["num_kv_heads"]
                # about half the workers read the cached positions: fewer,
                # larger splits merge faster (measured at batch 1: 16 splits
                # per kv head 3.82 ms, 32: 3.88 ms, 8: 3.90 ms), plus the
                # last split, which reads none and merges (17 at batch 1:
                # 3.582 against 3.611 ms for 16 with the merger reading its
                # share); the builder raises it to what the per-task block
                # budget needs and drops the extra split when the tasks would
                # outnumber the workers (batch 8: 5 splits x 64 > 256 workers
                # measured 5.92 against 5.05 ms for 4)
                splits = max(1, min(255, int(W // (self.ATTN_SPLIT_DIVISOR * per))))
                # (as the builder does: the cached-position splits the per-task
                # block budget needs, and the extra split only while every
                # attention task still gets a worker)
                # blocks per wave: 3, or more when the splits the cached
                # positions need would outnumber the workers (16 requests:
                # 2 splits of 5 blocks per wave on 256 workers instead of
                # 4 x 128 tasks, two per worker)
                bpw = 3
                while bpw < 16 and -(-self.max_seq_length // (7 * bpw * 64)) * per > W:
                    bpw += 1
                per_split = 7 * bpw * 64
                cached = max(splits, -(-self.max_seq_length // per_split))
                empty_merger = splits > 1 and (cached + 1) * per <= W
                splits = cached + 1 if empty_merger else cached
                # the mergers come last in the op's task list, so they sit on
                # consecutive workers, which the next linear op leaves free
                attn_free[l["output"].name] = per if empty_merger else 0
                ops.append(dict(type="attention", qkv=l["input"].name, k_cache=l["k_cache"].name,
                                v_cache=l["v_cache"].name, cos=l["cos"].name if l["cos"] is not None else None,
                                sin=l["sin"].name if l["sin"] is not None else None,
                                q_norm=l["q_norm"].name if l["q_norm"] is not None else None,
                                k_norm=l["k_norm"].name if l["k_norm"] is not None else None,
                                out=l["output"].name,
                                num_q_heads=l["num_q_heads"], num_kv_heads=l["num_kv_heads"],
                                head_dim=l["head_dim"], splits=splits, empty_merger=int(empty_merger),
                                blocks_per_wave=bpw))
                i += 1
                continue
            if k == "prepare_batch":
                ops.append(dict(type="prepare_batch"))
                i += 1
                continue
            raise YirageHipError(f"hip backend: layer '{k}' cannot be scheduled here (no fusion partner)")
        return ops

    _LINK_PRODUCERS = ("embed", "rmsnorm_linear", "linear", "rmsnorm_linear_silu", "attention")

    def _link_tensors(self):
        """Intermediate activations passed between tasks on different CUs are
        stored as 8-byte words {two bf16 values, 32-bit tag}: a consumer checks
        each word's tag against the producing op of this launch instead of
        waiting for the producer to confirm that its stores completed.  These
        are the kernel-owned tensors (new_tensor) written by embed / linear /
        attention ops; the logits of the argmax op stay plain bf16.  Storage is
        re-allocated here at twice the bf16 size.  Batch-1 graphs only."""
        if self.max_num_batched_tokens > 1:
            # every task re-reads all token rows of its input: at batch > 1
            # the doubled bytes cost more than the confirmation they replace
            # (measured at 8 tokens with only the residual stream linked, the
            # rows staged by all waves with tag checks: 5.46 against 5.18 ms)
            return
        owned = {id(t) for t in self._owned}
        for op in self.ops:
            if op["type"] not in self._LINK_PRODUCERS:
                continue
            t = self._tensors[op["out"]]
            if t.ll or t.tensor is None or id(t.tensor) not in owned or t.num_dims != 2 or t.dtype != bfloat16:
                continue
            buf = torch.zeros((t.dim(0), 2 * t.dim(1)), dtype=torch.bfloat16, device=t.tensor.device)
            self._owned[[id(x) for x in self._owned].index(id(t.tensor))] = buf
            owned.add(id(buf))
            t.tensor = buf
            t.ll = True

    def _graph_json(self) -> str:
        tensors = {}
        for t in self._tensors.values():
            if t.tensor is not None:
                ptr = 0 if t.tensor.device.type == "meta" else t.tensor.data_ptr()
                tensors[t.name] = dict(ptr=ptr, dims=list(t.dims), dtype=t.dtype, ll=int(t.ll))
        return json.dumps(dict(
            num_workers=self.num_workers, max_tokens=self.max_num_batched_tokens,
            max_requests=self.max_num_batched_requests, page_size=self.page_size, max_pages=self.max_num_pages,
            max_seq_len=self.max_seq_length, total_requests=self.total_num_requests,
            eos_token_id=int(self.eos_token_id), online=int(self.mode == "online"), tensors=tensors, ops=self.ops))

    # ------------------------------------------------------------ compile / run
    def compile(self, **kwargs):
        assert not self._is_compiled
        self.ops = self._fuse()
        self._link_tensors()
        g = ctypes.c_void_p()
        check(lib().yr_pk_graph_build(self._graph_json().encode(), ctypes.byref(g)), "task graph build")
        self._graph = g
        if kwargs.get("verify", True):
            rep = ctypes.create_string_buffer(1024)
            check(lib().yr_pk_graph_simulate(g, 1234, 2, kwargs.get("race_window", 8), rep, 1024),
                  "task graph simulation")
        if kwargs.get("build_only", False):
            # graph construction and verification only (no device resources)
            self._is_compiled = False
            return
        mt = self.meta_tensors
        m = _lib.PKMeta()
        for field_name, key in (("step", "step"), ("tokens", "tokens"), ("input_tokens", "input_tokens"),
                                ("output_tokens", "output_tokens"), ("num_new_tokens", "num_new_tokens"),
                                ("prompt_lengths", "prompt_lengths"), ("qo_indptr", "qo_indptr_buffer"),
                                ("paged_kv_indptr", "paged_kv_indptr_buffer"),
                                ("paged_kv_indices", "paged_kv_indices_buffer"),
                                ("paged_kv_last_page_len", "paged_kv_last_page_len_buffer")):
            t = mt.get(key)
            setattr(m, field_name, t.data_ptr() if t is not None else None)
        self._meta = m
        h = ctypes.c_void_p()
        check(lib().yr_pk_create(g, ctypes.byref(m), ctypes.byref(h)), "persistent kernel create")
        self._handle = h
        if self.max_num_batched_tokens > 1 and kwargs.get("pack_weights", True):
            # batch > 1: the linear tasks stream a copy of their weights laid
            # out in load order (about the linear weights' size again, in
            # HBM); pack_weights(False) frees it, pack_weights() after a
            # weight update refreshes it
            self.pack_weights(True)
        if any(o["type"] == "prepare_batch" for o in self.ops):
            check(lib().yr_pk_init_batch(h, self._stream()), "init batch")
        self._is_compiled = True
        if self.profiler_tensor is not None:
            self.enable_profiler(tensor=self.profiler_tensor)

    def _stream(self):
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def __call__(self, max_iterations: int | None = None, **kwargs):
        """Runs the task graph in one launch.  As the reference's offline
        ypk() (persistent_kernel.cuh:841-857, demo/llama3/demo.py:864-868),
        an offline kernel with a prepare_batch layer runs every step of the
        generation: the device starts the next pass while requests remain.
        Otherwise one pass (one step) per call.  `max_iterations` bounds the
        passes (0: until the batch is empty; needs prepare_batch)."""
        if not self._is_compiled:
            raise YirageHipError("PersistentKernel: call compile() first")
        if max_iterations is None:
            # offline: the whole generation; online (the host feeds each
            # step's accepted tokens through num_new_tokens) and onepass: one
            # pass per call, status()[1][1] says whether the sequence goes on
            has_prepare = any(o["type"] == "prepare_batch" for o in self.ops)
            max_iterations = 0 if (self.mode == "offline" and has_prepare) else 1
        check(lib().yr_pk_launch(self._handle, self._stream(), int(max_iterations)), "persistent kernel launch")
        if self.profiler_tensor is not None:
            # as the reference does after every launch (persistent_kernel.py:1322-1337)
            name = (self.trace_name or f"yirage_{self.mpi_rank}") + ".perfetto-trace"
            self.export_trace(name)

    def enable_profiler(self, enable: bool = True, tensor: torch.Tensor | None = None):
        """Per-task device timestamps (into `tensor`, int64 / uint64 with at
        least tasks x 8 entries, or a buffer allocated here); read them with
        profile() or export_trace()."""
        if enable:
            n = self.graph_info()["tasks"] * 8
            if tensor is None:
                tensor = torch.zeros(n, dtype=torch.int64, device="cuda")
            if tensor.dtype not in (torch.int64, torch.uint64) or tensor.numel() < n or not tensor.is_contiguous():
                raise YirageHipError(f"profiler tensor must be a contiguous int64 tensor of >= {n} entries")
            tensor.zero_()
            self._prof = tensor
            check(lib().yr_pk_set_profiler(self._handle, ctypes.c_void_p(self._prof.data_ptr()), n), "profiler")
        else:
            check(lib().yr_pk_set_profiler(self._handle, None, 0), "profiler")
            self._prof = None

    def profile(self):
        """[tasks, 8] int64 numpy array (10 ns ticks): start, inputs ready, end, worker,
        activations staged, compute done, outputs published (GEMV tasks), 0."""
        n = self.graph_info()["tasks"] * 8
        return self._prof.view(-1)[:n].view(-1, 8).cpu().numpy()

    def export_trace(self, file_name: str) -> int:
        """The last launch's per-task profile as a Perfetto trace (one track
        per worker, one slice per task); returns the number of slices."""
        from .profiler import export_to_perfetto_trace
        return export_to_perfetto_trace(self.profile(), file_name, self.task_table())

    def task_table(self):
        """[tasks, 10] int64: op, type, wait event, wait count, trigger event, row0, rows, i0, i1, i2."""
        if getattr(self, "_task_table", None) is None:
            n = self.graph_info()["tasks"]
            rec = (ctypes.c_int64 * 10)()
            import numpy as np
            out = np.zeros((n, 10), np.int64)
            for t in range(n):
                check(lib().yr_pk_graph_task(self._graph, t, rec, 10), "task")
                out[t] = list(rec)
            self._task_table = out
        return self._task_table.copy()

    def init_batch(self):
        """Reset the offline batch manager (request slots, page queue) on the
        device, as compile() does; the caller resets step / tokens."""
        check(lib().yr_pk_init_batch(self._handle, self._stream()), "init batch")

    def iterations(self) -> int:
        """Passes the last launch ran (synchronizes with the device)."""
        n = ctypes.c_int()
        check(lib().yr_pk_iterations(self._handle, ctypes.byref(n)), "iterations")
        return n.value

    def batch_state(self) -> dict:
        """The device batch manager's own state (synchronizes): request_ids,
        next_request_id, page_queue, page_queue_head, page_queue_tail."""
        import numpy as np
        MR, MP = self.max_num_batched_requests, self.max_num_pages
        buf = (ctypes.c_int * (MR + 3 + MP))()
        check(lib().yr_pk_read_batch(self._handle, buf, MR + 3 + MP), "read batch")
        a = np.array(buf, np.int32)
        return {"request_ids": a[:MR], "next_request_id": a[MR:MR + 1], "page_queue": a[MR + 1:MR + 1 + MP],
                "page_queue_head": a[MR + 1 + MP:MR + 2 + MP], "page_queue_tail": a[MR + 2 + MP:MR + 3 + MP]}

    def set_cooperative(self, cooperative: bool = True):
        """Cooperative (default) or ordinary launch of the worker grid."""
        check(lib().yr_pk_set_launch_mode(self._handle, int(bool(cooperative))), "launch mode")

    def pack_weights(self, enable: bool = True) -> int:
        """Batch > 1 graphs: give the linear tasks a copy of their weights in
        the order they stream them (sequential 1 KiB MFMA fragments instead
        of 16 rows x 64 bytes per load); False frees it.  Returns the bytes
        the copy holds (0 at batch 1, where rows already stream
        contiguously).  Results are bit-identical either way."""
        n = ctypes.c_size_t()
        check(lib().yr_pk_pack_weights(self._handle, int(bool(enable)), ctypes.byref(n)), "pack weights")
        return n.value

    def set_spin_limit(self, polls: int):
        """Watchdog: polls of one wait before the kernel gives up, flags
        status()[1][0] and drains (every later wait gives up at once)."""
        check(lib().yr_pk_set_spin_limit(self._handle, int(polls)), "spin limit")

    def reset_status(self):
        """After a watchdog exit: clear the status flags and re-base the
        event counters, arrival tickets and tagged words (synchronizes)."""
        check(lib().yr_pk_reset_status(self._handle), "reset status")

    def status(self):
        st = (ctypes.c_int * 4)()
        rc = lib().yr_pk_status(self._handle, st)
        return rc, list(st)

    def graph_info(self) -> dict:
        info = (ctypes.c_int64 * 8)()
        check(lib().yr_pk_graph_info(self._graph, info, 8), "graph info")
        keys = ("ops", "tasks", "events", "workers", "tickets", "scratch_floats", "max_queue")
        return dict(zip(keys, list(info)[:7]))

    def load_task_graph(self, graph, tensors: dict):
        """Record the layers of a task_graph.json (the reference's schema,
        src/kernel/runtime.cc:847-1318) on this kernel; compile() next."""
        from .task_graph import load_task_graph
        return load_task_graph(graph, self, tensors)

    def export_task_graph(self) -> str:
        """The compiled task graph in the reference's task_graph.json schema."""
        need = ctypes.c_size_t()
        check(lib().yr_pk_graph_export_json(self._graph, None, 0, ctypes.byref(need)), "export")
        buf = ctypes.create_string_buffer(need.value)
        check(lib().yr_pk_graph_export_json(self._graph, buf, need.value, None), "export")
        return buf.value.decode()

    def __del__(self):
        try:
            if not getattr(self, "__finalized__", True):
                self.finalize()
        except Exception:
            pass  # interpreter shutdown: the library may already be unloaded

    def finalize(self):
        if self.__finalized__:
            return
        if self._handle is not None:
            lib().yr_pk_destroy(self._handle)
            self._handle = None
        if self._graph is not None:
            lib().yr_pk_graph_free(self._graph)
            self._graph = None
        self.__finalized__ = True
