"""CPU round trip of task graphs in the reference's task_graph.json schema
(src/kernel/runtime.cc:847-1318): the Llama-3-8B persistent-kernel graph is
exported, loaded back into a fresh PersistentKernel with
yirage_amd.task_graph.load_task_graph and rebuilt; the rebuilt graph has the
same tasks, events and queues.  A graph written in the reference's own
vocabulary (separate rms_norm / linear / silu_mul / argmax tasks over fused
weight tensors) loads and builds too."""
import json

import numpy as np
import pytest
import torch

from yirage_amd.llama import LLAMA3_8B, LlamaConfig, LlamaDecodeModel
from yirage_amd.persistent_kernel import PersistentKernel
from yirage_amd.task_graph import load_task_graph


def _fresh_pk(model):
    return PersistentKernel(mode="offline", world_size=1, mpi_rank=0, num_workers=256, num_local_schedulers=0,
                            num_remote_schedulers=0, max_seq_length=model.max_seq,
                            max_num_batched_requests=model.MR, max_num_batched_tokens=model.MT,
                            max_num_pages=model.max_pages, page_size=model.page, eos_token_id=-1,
                            meta_tensors=model.meta)


def _binding(pk):
    out = {}
    for name, t in pk._tensors.items():
        if t.tensor is None or t.segments:
            continue
        # link tensors were re-allocated at twice the width; bind their logical shape
        out[name] = torch.empty(t.dims, dtype=t.tensor.dtype, device="meta") if t.ll else t.tensor
    return out


@pytest.mark.parametrize("batch", [1, 8])
def test_llama3_8b_task_graph_round_trip(batch):
    model = LlamaDecodeModel(LLAMA3_8B, batch=batch, kv_len=4096, device="meta")
    text = model.pk.export_task_graph()
    g = json.loads(text)
    info = model.pk.graph_info()
    # the reference's schema
    assert set(g) >= {"all_tasks", "all_events", "first_tasks"}
    assert len(g["all_tasks"]) == info["tasks"] + 2 and g["all_tasks"][0]["task_type"] == 0
    assert g["all_tasks"][1]["task_type"] == 10
    t = g["all_tasks"][2]
    assert set(t) >= {"task_type", "variant_id", "inputs", "outputs", "trigger_event", "dependent_event",
                      "request_id", "expert_offset"}
    assert set(t["inputs"][0]) == {"base_ptr", "offset", "data_type", "dims", "strides"}
    assert len(g["all_events"]) == info["events"]
    types = {x["task_type"] for x in g["all_tasks"]}
    assert {101, 102, 108, 116} <= types
    pk2 = _fresh_pk(model)
    load_task_graph(text, pk2, _binding(model.pk))
    pk2.compile(build_only=True)
    assert pk2.graph_info() == info
    assert np.array_equal(pk2.task_table(), model.pk.task_table())
    assert json.loads(pk2.export_task_graph())["all_events"] == g["all_events"]


def _reference_style_graph(cfg, T, names):
    """A task graph in the reference's vocabulary for a 1-layer model: separate
    rms_norm / linear / silu_mul / argmax tasks, weights as single (already
    fused / shuffled) tensors, as persistent_kernel.py + runtime.cc emit them."""
    H, D, G = cfg.hidden, cfg.head_dim, cfg.num_q_heads // cfg.num_kv_heads
    qkv_n = (cfg.num_q_heads + 2 * cfg.num_kv_heads) * D
    bf = 941

    def io(name, off, dims):
        strides = [dims[1], 1] if len(dims) == 2 else [1]
        return {"base_ptr": name, "offset": off * 2, "data_type": bf, "dims": list(dims), "strides": strides}

    tasks = [{"task_type": 0}, {"task_type": 10}]

    def linear(x, w, out, N, K, rpt, res=None, code=120):
        for r in range(0, N, rpt):
            ins = [io(x, 0, (T, K)), io(w, r * K, (rpt, K))]
            if res:
                ins.append(io(res, r, (T, rpt)))
            tasks.append({"task_type": code, "variant_id": 0, "inputs": ins, "outputs": [io(out, r, (T, rpt))]})

    tasks.append({"task_type": 101, "inputs": [{"base_ptr": "tok", "offset": 0, "data_type": 965, "dims": [T, 1],
                                                 "strides": [1, 1]}, io("embed", 0, (cfg.vocab, H))],
                  "outputs": [io("h0", 0, (T, H))]})
    tasks.append({"task_type": 119, "inputs": [io("h0", 0, (T, H)), io("ln1", 0, (H,))],
                  "outputs": [io("xn", 0, (T, H))]})
    linear("xn", "wqkv", "qkv", qkv_n, H, 64)
    for h in range(cfg.num_kv_heads):
        tasks.append({"task_type": 116, "inputs": [io("qkv", h * (G + 2) * D, (T, (G + 2) * D)),
                                                     {"base_ptr": "kc", "offset": 0, "data_type": bf, "dims": [1],
                                                      "strides": [1]},
                                                     {"base_ptr": "vc", "offset": 0, "data_type": bf, "dims": [1],
                                                      "strides": [1]}, io("cos", 0, (64, D)), io("sin", 0, (64, D))],
                      "outputs": [io("att", h * G * D, (T, G * D))], "request_id": 0})
    linear("att", "wo", "h1", H, cfg.num_q_heads * D, 64, res="h0", code=108)
    tasks.append({"task_type": 119, "inputs": [io("h1", 0, (T, H)), io("ln2", 0, (H,))],
                  "outputs": [io("xn", 0, (T, H))]})
    linear("xn", "wgu", "mid", 2 * cfg.intermediate, H, 64)
    for r in range(0, cfg.intermediate, 32):
        tasks.append({"task_type": 118, "inputs": [io("mid", 2 * r, (T, 64))], "outputs": [io("act", r, (T, 32))]})
    linear("act", "wd", "h2", H, cfg.intermediate, 64, res="h1", code=108)
    tasks.append({"task_type": 119, "inputs": [io("h2", 0, (T, H)), io("lnf", 0, (H,))],
                  "outputs": [io("xn", 0, (T, H))]})
    linear("xn", "lm", "logits", cfg.vocab, H, 128)
    tasks.append({"task_type": 110, "inputs": [io("logits", 0, (T, cfg.vocab))], "outputs": []})
    tasks.append({"task_type": 111, "inputs": [], "outputs": [{"base_ptr": "out_tok", "offset": 0,
                                                                "data_type": 965, "dims": [T, 1], "strides": [1, 1]}]})
    return {"all_tasks": tasks, "all_events": [], "first_tasks": [2]}


def test_reference_vocabulary_graph_loads_and_builds():
    cfg = LlamaConfig(num_layers=1, hidden=1024, num_q_heads=8, num_kv_heads=2, intermediate=2048, vocab=4096)
    model = LlamaDecodeModel(cfg, batch=1, kv_len=100, device="meta")
    T, H, D = 1, cfg.hidden, cfg.head_dim
    bf, m = torch.bfloat16, "meta"
    qkv_n = (cfg.num_q_heads + 2 * cfg.num_kv_heads) * D
    tens = {
        "tok": model.meta["input_tokens"], "embed": torch.empty((cfg.vocab, H), dtype=bf, device=m),
        "ln1": torch.empty(H, dtype=bf, device=m), "ln2": torch.empty(H, dtype=bf, device=m),
        "lnf": torch.empty(H, dtype=bf, device=m),
        "wqkv": torch.empty((qkv_n, H), dtype=bf, device=m),
        "wo": torch.empty((H, cfg.num_q_heads * D), dtype=bf, device=m),
        "wgu": torch.empty((2 * cfg.intermediate, H), dtype=bf, device=m),
        "wd": torch.empty((H, cfg.intermediate), dtype=bf, device=m),
        "lm": torch.empty((cfg.vocab, H), dtype=bf, device=m),
        "kc": model.kc[0], "vc": model.vc[0], "cos": model.cos, "sin": model.sin,
        "out_tok": model.meta["output_tokens"],
    }
    for n, shp in (("h0", (8, H)), ("xn", (8, H)), ("qkv", (8, qkv_n)), ("att", (8, cfg.num_q_heads * D)),
                   ("h1", (8, H)), ("mid", (8, 2 * cfg.intermediate)), ("act", (8, cfg.intermediate)),
                   ("h2", (8, H)), ("logits", (8, cfg.vocab))):
        tens[n] = torch.empty(shp, dtype=bf, device=m)
    pk = _fresh_pk(model)
    load_task_graph(_reference_style_graph(cfg, T, tens), pk, tens)
    pk.compile(build_only=True)
    kinds = [op["type"] for op in pk.ops]
    assert kinds == ["embed", "rmsnorm_linear", "attention", "linear", "rmsnorm_linear_silu", "linear",
                     "rmsnorm_linear_argmax"]
    silu = pk.ops[4]
    assert silu["group"] == 32 and silu["weight"] == [("wgu", 0, 2 * cfg.intermediate)]


def test_qk_norm_graph_round_trip():
    """paged_attention_layer(q_norm=..., k_norm=...): the export lists the
    reference's operand order (input, k_cache, v_cache, q_norm, k_norm, cos,
    sin) and re-imports to the same tasks; the op carries the qk-norm flag."""
    cfg = LlamaConfig(num_layers=2, hidden=1024, num_q_heads=8, num_kv_heads=2, intermediate=2048, vocab=4096,
                      qk_norm=True)
    model = LlamaDecodeModel(cfg, batch=1, kv_len=100, device="meta")
    att = [o for o in model.pk.ops if o["type"] == "attention"]
    assert att and all(o["q_norm"] and o["k_norm"] for o in att)
    text = model.pk.export_task_graph()
    g = json.loads(text)
    pa = [t for t in g["all_tasks"] if t["task_type"] == 116]
    assert pa and [len(t["inputs"]) for t in pa[:1]] == [7]
    assert pa[0]["inputs"][3]["dims"] == [cfg.head_dim] and pa[0]["inputs"][4]["dims"] == [cfg.head_dim]
    pk2 = _fresh_pk(model)
    load_task_graph(text, pk2, _binding(model.pk))
    pk2.compile(build_only=True)
    assert np.array_equal(pk2.task_table(), model.pk.task_table())
    assert [o.get("q_norm") for o in pk2.ops if o["type"] == "attention"] == [o["q_norm"] for o in att]
