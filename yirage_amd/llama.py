"""Llama-3-shaped decode step on the persistent kernel.

Builds the same layer sequence as the reference demo
(demo/llama3/demo.py:472-812): embedding -> per layer [rmsnorm, QKV linear
over per-kv-group shuffled weights, paged attention with RoPE, O linear with
residual, rmsnorm, gate/up linear over shuffled weights, silu_mul, down
linear with residual] -> final rmsnorm -> LM head -> argmax partial/reduce.
Weights are random-init (deterministic counter-hash ~N(0, 0.02), RMSNorm
weights 1.0), generated on the device; the KV cache is prefilled with
~N(0, 1) values behind a seeded random page table.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import fused
from .persistent_kernel import PersistentKernel, bfloat16, int64


@dataclass
class LlamaConfig:
    num_layers: int = 32
    hidden: int = 4096
    num_q_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 14336
    vocab: int = 128256
    rope_theta: float = 500000.0
    eps: float = 1e-6        # the reference MPK rmsnorm task uses 1e-6 (task_register.cc:118-122)
    weight_std: float = 0.02
    qk_norm: bool = False    # per-head RMSNorm of q and k before RoPE (Qwen3-style; paged_attention_layer q_norm/k_norm)

    @property
    def qkv_out(self) -> int:
        return (self.num_q_heads + 2 * self.num_kv_heads) * self.head_dim

    def param_count(self) -> int:
        h, i, kv = self.hidden, self.intermediate, self.num_kv_heads * self.head_dim
        per_layer = h * (self.num_q_heads * self.head_dim) + 2 * h * kv + (self.num_q_heads * self.head_dim) * h \
            + 3 * h * i + 2 * h
        return self.num_layers * per_layer + self.vocab * h + h  # + LM head + final norm (embedding separate)


LLAMA3_8B = LlamaConfig()

# tensor ids for the deterministic generator: seed = base * 1000 + layer * 16 + id
_IDS = {"wq": 1, "wk": 2, "wv": 3, "wo": 4, "wg": 5, "wu": 6, "wd": 7, "kc": 8, "vc": 9, "qn": 10, "kn": 11}
QK_NORM_STD = 0.1  # qk-norm weights: 1 + N(0, 0.1), rounded to bf16


def tensor_seed(base: int, layer: int, name: str) -> int:
    if name == "embed":
        return base * 1000 + 999_000
    if name == "lm_head":
        return base * 1000 + 999_001
    return base * 1000 + layer * 16 + _IDS[name]


def weight_shapes(cfg: LlamaConfig) -> dict:
    h, d = cfg.hidden, cfg.head_dim
    return {"wq": (cfg.num_q_heads * d, h), "wk": (cfg.num_kv_heads * d, h), "wv": (cfg.num_kv_heads * d, h),
            "wo": (h, cfg.num_q_heads * d), "wg": (cfg.intermediate, h), "wu": (cfg.intermediate, h),
            "wd": (h, cfg.intermediate)}


def rope_tables(max_pos: int, head_dim: int, theta: float):
    """Llama rotate-half cos/sin tables [pos, head_dim], rounded to bf16
    (the reference feeds rotary_emb outputs, demo.py:180-181)."""
    inv = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim))
    ang = np.outer(np.arange(max_pos, dtype=np.float64), inv)
    emb = np.concatenate([ang, ang], -1)
    return (torch.from_numpy(np.cos(emb)).to(torch.bfloat16), torch.from_numpy(np.sin(emb)).to(torch.bfloat16))


def page_table(batch: int, kv_len: int, page: int, seed: int):
    """Random page table: every sequence owns ceil(kv_len / page) pages drawn
    from a seeded permutation of the pool; returns (indptr, indices, pool)."""
    npg = (kv_len + page - 1) // page
    pool = batch * npg
    perm = np.random.default_rng(seed).permutation(pool).astype(np.int32)
    indptr = (np.arange(batch + 1) * npg).astype(np.int32)
    return indptr, perm, pool


class LlamaDecodeModel:
    """Random-init weights + KV cache on the device and a PersistentKernel.

    Decode mode (prompts=None): `batch` requests of one new token each over a
    KV cache prefilled to kv_len positions; every launch repeats that step.

    Serving mode (prompts = list of token-id lists, with_prepare=True): the
    offline batch manager of the reference (prepare_next_batch,
    persistent_kernel.cuh:169-322) runs as the graph's last task and schedules
    prefill chunks and decode steps of the requests over max_requests slots
    and max_tokens rows per launch, allocating KV pages from a FIFO queue."""

    def __init__(self, cfg: LlamaConfig, batch: int, kv_len: int = 0, page_size: int = 64, seed: int = 0,
                 num_workers: int | None = None, with_prepare: bool = False, device="cuda", prompts=None,
                 max_tokens: int | None = None, max_requests: int | None = None, max_seq: int | None = None,
                 eos_token_id: int = -1, mode: str = "offline"):
        self.cfg, self.batch, self.kv_len, self.page, self.seed = cfg, batch, kv_len, page_size, seed
        self.MR = max_requests or batch
        self.MT = max_tokens or batch
        self.eos = eos_token_id
        self.mode = mode
        serving = prompts is not None
        if serving and not with_prepare:
            raise ValueError("serving mode needs the batch manager (with_prepare=True)")
        dev = torch.device(device)
        self.graph_only = dev.type == "meta"   # build/verify the task graph without a GPU
        fill = (lambda t, seed, std: t) if self.graph_only else fused.synth_fill
        bf = torch.bfloat16
        H = cfg.hidden
        self.w = []
        for layer in range(cfg.num_layers):
            lw = {}
            for name, shp in weight_shapes(cfg).items():
                t = torch.empty(shp, dtype=bf, device=dev)
                fill(t, tensor_seed(seed, layer, name), cfg.weight_std)
                lw[name] = t
            if cfg.qk_norm:
                for name in ("qn", "kn"):
                    t = torch.empty(cfg.head_dim, dtype=bf, device=dev)
                    fill(t, tensor_seed(seed, layer, name), QK_NORM_STD)
                    lw[name] = t if self.graph_only else (1.0 + t.float()).to(bf)
            lw["ln1"] = torch.ones(H, dtype=bf, device=dev)
            lw["ln2"] = torch.ones(H, dtype=bf, device=dev)
            self.w.append(lw)
        self.embed = fill(torch.empty((cfg.vocab, H), dtype=bf, device=dev), tensor_seed(seed, 0, "embed"),
                          cfg.weight_std)
        self.lm_head = fill(torch.empty((cfg.vocab, H), dtype=bf, device=dev), tensor_seed(seed, 0, "lm_head"),
                            cfg.weight_std)
        self.final_norm = torch.ones(H, dtype=bf, device=dev)
        if serving:
            self.max_seq = max_seq or (max(len(p) for p in prompts) + 16)
            npg = (self.max_seq + page_size - 1) // page_size
            pool = self.MR * npg
            indptr = np.zeros(self.MR + 1, np.int32)
            indices = np.zeros(pool, np.int32)
        else:
            indptr, indices, pool = page_table(batch, kv_len, page_size, seed + 7)
            self.max_seq = kv_len + 8
        # paged KV cache (prefilled with ~N(0, 1) in decode mode; in serving
        # mode every position is written before it is read)
        self.max_pages = pool
        self.kc, self.vc = [], []
        for layer in range(cfg.num_layers):
            shp = (pool, page_size, cfg.num_kv_heads, cfg.head_dim)
            self.kc.append(fill(torch.empty(shp, dtype=bf, device=dev), tensor_seed(seed, layer, "kc"), 1.0))
            self.vc.append(fill(torch.empty(shp, dtype=bf, device=dev), tensor_seed(seed, layer, "vc"), 1.0))
        cos, sin = rope_tables(max(self.max_seq, 64), cfg.head_dim, cfg.rope_theta)
        self.cos, self.sin = cos.to(dev), sin.to(dev)
        # meta tensors (python/yirage/persistent_kernel.py:268-279)
        i32, i64 = torch.int32, torch.int64
        if serving:
            R = len(prompts)
            tokens = torch.zeros((R, self.max_seq), dtype=i64)
            for i, p in enumerate(prompts):
                tokens[i, :len(p)] = torch.as_tensor(p, dtype=i64)
            self.meta = {
                "step": torch.zeros((R,), dtype=i32, device=dev),
                "tokens": tokens.to(dev),
                "input_tokens": torch.zeros((self.MT, 1), dtype=i64, device=dev),
                "output_tokens": torch.zeros((self.MT, 1), dtype=i64, device=dev),
                "num_new_tokens": torch.zeros((R,), dtype=i32, device=dev),
                "prompt_lengths": torch.tensor([len(p) for p in prompts], dtype=i32, device=dev),
                "qo_indptr_buffer": torch.zeros(self.MR + 1, dtype=i32, device=dev),
                "paged_kv_indptr_buffer": torch.zeros(self.MR + 1, dtype=i32, device=dev),
                "paged_kv_indices_buffer": torch.zeros(pool, dtype=i32, device=dev),
                "paged_kv_last_page_len_buffer": torch.zeros(self.MR, dtype=i32, device=dev),
            }
        else:
            lpl = kv_len % page_size
            self.meta = {
                "step": torch.full((batch,), kv_len - 1, dtype=i32, device=dev),
                "tokens": torch.zeros((batch, self.max_seq), dtype=i64, device=dev),
                "input_tokens": torch.zeros((max(8, self.MT), 1), dtype=i64, device=dev),
                "output_tokens": torch.zeros((max(8, self.MT), 1), dtype=i64, device=dev),
                "num_new_tokens": torch.ones((batch,), dtype=i32, device=dev),
                "prompt_lengths": torch.full((batch,), kv_len - 1, dtype=i32, device=dev),
                "qo_indptr_buffer": torch.arange(batch + 1, dtype=i32, device=dev),
                "paged_kv_indptr_buffer": torch.from_numpy(indptr).to(dev),
                "paged_kv_indices_buffer": torch.from_numpy(indices).to(dev),
                "paged_kv_last_page_len_buffer": torch.full((batch,), lpl, dtype=i32, device=dev),
            }
        self.page_indptr, self.page_indices = indptr, indices
        keep = {k: v.clone() for k, v in self.meta.items()} if (mode == "online" and not serving) else None
        self.pk = self._build(num_workers, with_prepare)
        if keep is not None and not self.graph_only:
            # the batch reset at compile (init_kernel of the reference) clears
            # the page table; in online mode the host owns it: restore it
            for k, v in keep.items():
                self.meta[k].copy_(v)

    def _build(self, num_workers, with_prepare):
        cfg, B = self.cfg, self.MT  # activation rows = tokens per launch
        if num_workers is None:
            num_workers = 256 if self.graph_only else torch.cuda.get_device_properties(0).multi_processor_count
        pk = PersistentKernel(mode=self.mode, world_size=1, mpi_rank=0, num_workers=num_workers,
                              num_local_schedulers=0, num_remote_schedulers=0, max_seq_length=self.max_seq,
                              max_num_batched_requests=self.MR, max_num_batched_tokens=self.MT,
                              max_num_pages=self.max_pages, page_size=self.page, eos_token_id=self.eos,
                              meta_tensors=self.meta)
        pk.vocab_size = cfg.vocab
        H = cfg.hidden
        x = pk.attach_input(self.meta["input_tokens"], name="input_token")
        cos = pk.attach_input(self.cos, name="cos_position_embedding")
        sin = pk.attach_input(self.sin, name="sin_position_embedding")
        embed_w = pk.attach_input(self.embed, name="embed_tokens")
        t = {}
        t["embed_out"] = pk.new_tensor((B, H), dtype=bfloat16, name="embed_out")
        t["rmsnorm_out"] = pk.new_tensor((B, H), dtype=bfloat16, name="rmsnorm_out")
        t["attn_in"] = pk.new_tensor((B, cfg.qkv_out), dtype=bfloat16, name="attn_in")
        t["attn_out"] = pk.new_tensor((B, cfg.num_q_heads * cfg.head_dim), dtype=bfloat16, name="attn_out")
        t["attn_proj_out"] = pk.new_tensor((B, H), dtype=bfloat16, name="attn_proj_out")
        t["mlp_mid"] = pk.new_tensor((B, 2 * cfg.intermediate), dtype=bfloat16, name="mlp_mid")
        t["silu_mul_out"] = pk.new_tensor((B, cfg.intermediate), dtype=bfloat16, name="silu_mul_out")
        t["mlp_out"] = pk.new_tensor((B, H), dtype=bfloat16, name="mlp_out")
        t["argmax_in"] = pk.new_tensor((B, cfg.vocab), dtype=bfloat16, name="argmax_in")
        t["argmax_part_value"] = pk.new_tensor((B, num_workers), dtype=bfloat16, name="argmax_part_value")
        t["argmax_part_index"] = pk.new_tensor((B, num_workers), dtype=int64, name="argmax_part_index")
        out_tok = pk.attach_input(self.meta["output_tokens"], name="output_token")
        pk.embed_layer(input=x, weight=embed_w, output=t["embed_out"], grid_dim=(1, 1, 1), block_dim=(128, 1, 1),
                       input_source=1)
        h = t["embed_out"]
        for i in range(cfg.num_layers):
            lw = self.w[i]
            w_norm = pk.attach_input(lw["ln1"], name=f"layer_{i}_input_layernorm")
            wq = pk.attach_input(lw["wq"], name=f"layer_{i}_q_proj")
            wk = pk.attach_input(lw["wk"], name=f"layer_{i}_k_proj")
            wv = pk.attach_input(lw["wv"], name=f"layer_{i}_v_proj")
            w_qkv = pk.shuffle_tensors([wq, wk, wv], 0, cfg.num_kv_heads, name=f"layer_{i}_qkv_proj")
            pk.rmsnorm_layer(input=h, weight=w_norm, output=t["rmsnorm_out"], grid_dim=(B, 1, 1), block_dim=(128, 1, 1))
            pk.linear_layer(input=t["rmsnorm_out"], weight=w_qkv, output=t["attn_in"], grid_dim=(96, 1, 1),
                            block_dim=(128, 1, 1))
            kc = pk.attach_input(self.kc[i], name=f"layer_{i}_k_cache")
            vc = pk.attach_input(self.vc[i], name=f"layer_{i}_v_cache")
            qn = kn = None
            if cfg.qk_norm:
                qn = pk.attach_input(lw["qn"], name=f"layer_{i}_q_norm")
                kn = pk.attach_input(lw["kn"], name=f"layer_{i}_k_norm")
            pk.paged_attention_layer(input=t["attn_in"], k_cache=kc, v_cache=vc, q_norm=qn, k_norm=kn,
                                     cos_pos_embed=cos, sin_pos_embed=sin, output=t["attn_out"],
                                     grid_dim=(self.MR, cfg.num_kv_heads, 1), block_dim=(128, 1, 1))
            wo = pk.attach_input(lw["wo"], name=f"layer_{i}_o_proj")
            pk.linear_with_residual_layer(input=t["attn_out"], weight=wo, residual=h, output=t["attn_proj_out"],
                                          grid_dim=(H // 64, 1, 1), block_dim=(128, 1, 1))
            h = t["attn_proj_out"]
            w_norm2 = pk.attach_input(lw["ln2"], name=f"layer_{i}_post_attn_layernorm")
            wg = pk.attach_input(lw["wg"], name=f"layer_{i}_gate_proj")
            wu = pk.attach_input(lw["wu"], name=f"layer_{i}_up_proj")
            groups = num_workers if cfg.intermediate % num_workers == 0 else cfg.intermediate // 64
            w_gu = pk.shuffle_tensors([wg, wu], 0, groups, name=f"layer_{i}_gatedup_proj")
            pk.rmsnorm_layer(input=h, weight=w_norm2, output=t["rmsnorm_out"], grid_dim=(B, 1, 1), block_dim=(128, 1, 1))
            pk.linear_layer(input=t["rmsnorm_out"], weight=w_gu, output=t["mlp_mid"], grid_dim=(112, 1, 1),
                            block_dim=(128, 1, 1))
            pk.silu_mul_layer(input=t["mlp_mid"], output=t["silu_mul_out"], grid_dim=(56, 1, 1), block_dim=(128, 1, 1))
            wd = pk.attach_input(lw["wd"], name=f"layer_{i}_down_proj")
            out = t["mlp_out"]
            pk.linear_with_residual_layer(input=t["silu_mul_out"], weight=wd, residual=h, output=out,
                                          grid_dim=(H // 64, 1, 1), block_dim=(128, 1, 1))
            h = out
        w_norm = pk.attach_input(self.final_norm, name="model_norm_weight")
        w_proj = pk.attach_input(self.lm_head, name="lm_head")
        pk.rmsnorm_layer(input=h, weight=w_norm, output=t["rmsnorm_out"], grid_dim=(B, 1, 1), block_dim=(128, 1, 1))
        pk.linear_layer(input=t["rmsnorm_out"], weight=w_proj, output=t["argmax_in"], grid_dim=(501, 1, 1),
                        block_dim=(128, 1, 1))
        pk.argmax_partial_layer(input=t["argmax_in"], output=(t["argmax_part_value"], t["argmax_part_index"]),
                                grid_dim=(num_workers, 1, 1), block_dim=(128, 1, 1))
        pk.argmax_reduce_layer(input=(t["argmax_part_value"], t["argmax_part_index"]), output=out_tok,
                               grid_dim=(1, 1, 1), block_dim=(128, 1, 1))
        if with_prepare:
            pk.prepare_batch_layer()
        self.t = t
        pk.compile(build_only=self.graph_only)
        return pk

    def set_input_tokens(self, ids):
        ids = torch.as_tensor(ids, dtype=torch.int64).view(-1, 1)
        self.meta["input_tokens"][: ids.shape[0]].copy_(ids.to(self.meta["input_tokens"].device))

    def step(self):
        """One decode / extend step (one task-graph pass)."""
        self.pk(max_iterations=1)

    def generate(self, max_iterations: int = 0):
        """Serving mode: every remaining step in one launch (0: until every
        request finished); returns the passes the device ran."""
        self.pk(max_iterations=max_iterations)
        return self.pk.iterations()

    def weight_bytes(self) -> int:
        """Bytes one decode step streams from weights (LM head and all layer
        matrices; the embedding contributes only the gathered rows)."""
        cfg = self.cfg
        return 2 * (cfg.param_count())

    def kv_bytes(self) -> int:
        cfg = self.cfg
        return self.batch * cfg.num_layers * 2 * self.kv_len * cfg.num_kv_heads * cfg.head_dim * 2
