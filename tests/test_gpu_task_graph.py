"""GPU run of a task graph written in the reference's task_graph.json
vocabulary (src/kernel/runtime.cc:847-1318: separate rms_norm / linear /
linear_with_residual / paged_attention / silu_mul / argmax tasks over fused
weight tensors, as python/yirage/persistent_kernel.py + runtime.cc emit
them), loaded with yirage_amd.task_graph.load_task_graph onto real device
tensors, compiled for this backend and launched.  The decode step it runs
must match the CPU oracle composition (tests/llama_oracle.decode_step):
logits within 2e-2 * max(1, max|logit|), the argmax token equal unless a
near-tie.  A wrong row offset, a wrong [gate | up] group or QKV shuffle
remap in the importer would move the logits far outside that bound.

The graph is the 8B exporter's too: the full-size export of this backend's
own graph is loaded back and run, and must reproduce the original kernel's
logits bit for bit."""
import json

import numpy as np
import pytest
import torch

from tests.llama_oracle import decode_step
from tests.test_task_graph import _binding, _fresh_pk, _reference_style_graph
from yirage_amd.llama import LlamaConfig, LlamaDecodeModel
from yirage_amd.task_graph import load_task_graph

pytestmark = pytest.mark.gpu


def _values(t):
    """Logical [rows, cols] bf16 values of a kernel tensor (a link tensor
    stores each bf16 pair with a 32-bit tag in one 8-byte word)."""
    if not t.ll:
        return t.tensor
    rows, cols = t.dims
    return t.tensor.view(rows, cols // 2, 4)[..., :2].reshape(rows, cols)


def _device_binding(pk):
    """Name -> tensor for re-import; link tensors get plain device tensors of
    their logical shape (the new kernel allocates nothing for bound names)."""
    out = _binding(pk)
    for name, t in pk._tensors.items():
        if name in out and t.ll:
            out[name] = torch.zeros(t.dims, dtype=torch.bfloat16, device="cuda")
    return out


def test_reference_vocabulary_graph_runs():
    cfg = LlamaConfig(num_layers=1, hidden=1024, num_q_heads=8, num_kv_heads=2, intermediate=2048, vocab=4096)
    seed, kv_len = 3, 100
    print("case reference-vocabulary task graph, 1 layer, B=1 kv=100", flush=True)
    model = LlamaDecodeModel(cfg, batch=1, kv_len=kv_len, seed=seed)
    H, D, G = cfg.hidden, cfg.head_dim, cfg.num_q_heads // cfg.num_kv_heads
    lw = model.w[0]
    # fused weights as the reference's shuffle_tensors / fuse_tensors lay them out
    rows = []
    for g in range(cfg.num_kv_heads):
        rows += [lw["wq"][g * G * D:(g + 1) * G * D], lw["wk"][g * D:(g + 1) * D], lw["wv"][g * D:(g + 1) * D]]
    wqkv = torch.cat(rows, 0).contiguous()
    gu = []
    for r in range(0, cfg.intermediate, 32):  # silu_mul tasks read [gate 32 | up 32] per 32 outputs
        gu += [lw["wg"][r:r + 32], lw["wu"][r:r + 32]]
    wgu = torch.cat(gu, 0).contiguous()
    bf, dev = torch.bfloat16, "cuda"
    qkv_n = (cfg.num_q_heads + 2 * cfg.num_kv_heads) * D
    tens = {
        "tok": model.meta["input_tokens"], "embed": model.embed, "ln1": lw["ln1"], "ln2": lw["ln2"],
        "lnf": model.final_norm, "wqkv": wqkv, "wo": lw["wo"], "wgu": wgu, "wd": lw["wd"], "lm": model.lm_head,
        "kc": model.kc[0], "vc": model.vc[0], "cos": model.cos, "sin": model.sin,
        "out_tok": model.meta["output_tokens"],
    }
    for n, shp in (("h0", (8, H)), ("xn", (8, H)), ("qkv", (8, qkv_n)), ("att", (8, cfg.num_q_heads * D)),
                   ("h1", (8, H)), ("mid", (8, 2 * cfg.intermediate)), ("act", (8, cfg.intermediate)),
                   ("h2", (8, H)), ("logits", (8, cfg.vocab))):
        tens[n] = torch.zeros(shp, dtype=bf, device=dev)
    pk = _fresh_pk(model)
    load_task_graph(_reference_style_graph(cfg, 1, tens), pk, tens)
    pk.compile()
    tokens = np.array([1234])
    model.set_input_tokens(tokens)
    pk(max_iterations=1)
    torch.cuda.synchronize()
    rc, st = pk.status()
    assert rc == 0, st
    ref_logits, ref_ids = decode_step(cfg, 1, kv_len, 64, seed, tokens)
    got = _values(pk._tensors["logits"]).float().cpu().numpy()[:1, :cfg.vocab]
    err = np.abs(got - ref_logits)
    print(f"  logits max abs err {err.max():.4f} (max |logit| {np.abs(ref_logits).max():.3f})", flush=True)
    assert err.max() <= 2e-2 * max(1.0, float(np.abs(ref_logits).max())), "imported graph's logits differ"
    tok = int(model.meta["output_tokens"][0, 0])
    if tok != int(ref_ids[0]):
        top = np.sort(ref_logits[0])[-2:]
        assert top[1] - top[0] <= 2 ** -7 * max(abs(top[1]), 1e-3), f"token {tok} != {ref_ids[0]}"
    pk.finalize()


def test_exported_graph_reimported_runs_bit_identical():
    cfg = LlamaConfig(num_layers=2, hidden=1024, num_q_heads=8, num_kv_heads=2, intermediate=2048, vocab=4096)
    print("case export -> import -> run, 2 layers, B=3 kv=130", flush=True)
    model = LlamaDecodeModel(cfg, batch=3, kv_len=130, seed=5)
    model.set_input_tokens([7, 99, 4000])
    kc0 = [k.clone() for k in model.kc]
    vc0 = [v.clone() for v in model.vc]
    model.step()
    torch.cuda.synchronize()
    assert model.pk.status()[0] == 0
    assert not model.t["argmax_in"].ll  # batch 3: plain activations
    want = model.t["argmax_in"].tensor.clone()
    want_tok = model.meta["output_tokens"].clone()
    text = model.pk.export_task_graph()
    assert json.loads(text)["all_tasks"][0]["task_type"] == 0
    # restore the caches (the step appended its token) and run the re-imported graph
    for i in range(cfg.num_layers):
        model.kc[i].copy_(kc0[i])
        model.vc[i].copy_(vc0[i])
    model.t["argmax_in"].tensor.zero_()
    model.meta["output_tokens"].zero_()
    pk2 = _fresh_pk(model)
    binding = _device_binding(model.pk)
    assert all(t.device.type == "cuda" for t in binding.values())
    load_task_graph(text, pk2, binding)
    pk2.compile()
    pk2(max_iterations=1)
    torch.cuda.synchronize()
    assert pk2.status()[0] == 0
    got = _values(pk2._tensors["argmax_in"])
    assert torch.equal(got[:3], want[:3]), "re-imported logits differ"
    assert torch.equal(model.meta["output_tokens"], want_tok)
    pk2.finalize()
