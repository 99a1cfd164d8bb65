"""GPU parity of the persistent megakernel (Llama-3-shaped decode step)
against the CPU oracle composition in tests/llama_oracle.py.

Logits of stacks of up to two layers must lie within 2e-2 * max(1, max|logit|)
of the oracle element-wise; the 32-layer step is bounded in relative L2.  The
argmax token ids must match exactly unless the oracle's top-2 logits are
within one bf16 ulp of each other (a near-tie, reported for that row)."""
import numpy as np
import pytest
import torch

from tests.llama_oracle import decode_step
from yirage_amd.llama import LlamaConfig, LlamaDecodeModel

pytestmark = pytest.mark.gpu


def _check(model, tokens, ref_logits, ref_ids, what, rel_l2=None, elementwise=False):
    got = model.t["argmax_in"].tensor.float().cpu().numpy()[: model.batch]
    ids = model.meta["output_tokens"].cpu().numpy().reshape(-1)[: model.batch]
    err = np.abs(got - ref_logits)
    scale = np.abs(ref_logits).max()
    print(f"[{what}] logits max abs err {err.max():.4f} (max |logit| {scale:.3f}), ids {ids.tolist()} "
          f"ref {ref_ids.tolist()}", flush=True)
    if elementwise:
        # the north-star tolerance, element by element (only where the
        # model's own rounding noise stays below it: one layer).  At batch 8
        # the oracle's own noise floor (tests/test_oracle.py::
        # test_logit_noise_floor_llama3_8b_one_layer_batch8) puts up to 0.1 %
        # of the logits outside it, none by more than 2^-5
        bad = err > 1e-2 + 1e-2 * np.abs(ref_logits)
        print(f"  element-wise rtol/atol 1e-2: {bad.sum()} of {bad.size} outside", flush=True)
        if model.batch == 1:
            assert not bad.any(), f"{what}: logits outside rtol/atol 1e-2"
        else:
            assert bad.mean() <= 1e-3, f"{what}: {bad.sum()} logits outside rtol/atol 1e-2"
            assert err.max() <= 2.0 ** -5 + 1e-6, f"{what}: a logit moved by {err.max()}"
    if rel_l2 is None:
        assert err.max() <= 2e-2 * max(1.0, scale), f"{what}: logits differ"
    else:
        # deep stacks: one bf16 rounding flip in the residual stream spreads
        # through every later layer, so the bound is on the relative L2 error
        r = np.linalg.norm(got - ref_logits) / np.linalg.norm(ref_logits)
        print(f"  relative L2 error {r:.3e}", flush=True)
        assert r <= rel_l2, f"{what}: logits differ (relative L2 {r})"
    for b in range(model.batch):
        top = np.sort(ref_logits[b])[-2:]
        if ids[b] != ref_ids[b]:
            gap = top[1] - top[0]
            assert gap <= 2 ** -7 * max(abs(top[1]), 1e-3), f"{what}: token {b} differs (gap {gap})"
            print(f"  near-tie at row {b}: gap {gap}", flush=True)


@pytest.mark.parametrize("batch,kv_len,qk_norm", [(1, 200, False), (3, 130, False), (8, 64, False),
                                                  (1, 200, True), (3, 130, True), (16, 100, False),
                                                  (12, 70, True)])
def test_small_llama_decode_step(batch, kv_len, qk_norm):
    """qk_norm: per-head RMSNorm of q and the new k before RoPE
    (paged_attention_layer(q_norm=..., k_norm=...))."""
    cfg = LlamaConfig(num_layers=2, hidden=1024, num_q_heads=8, num_kv_heads=2, head_dim=128, intermediate=2048,
                      vocab=4096, qk_norm=qk_norm)
    print(f"case small llama B={batch} kv={kv_len} qk_norm={qk_norm}", flush=True)
    model = LlamaDecodeModel(cfg, batch=batch, kv_len=kv_len, seed=3)
    tokens = (np.arange(batch) * 37 + 11) % cfg.vocab
    model.set_input_tokens(tokens)
    model.step()
    torch.cuda.synchronize()
    rc, st = model.pk.status()
    assert rc == 0, st
    ref_logits, ref_ids = decode_step(cfg, batch, kv_len, 64, 3, tokens)
    _check(model, tokens, ref_logits, ref_ids, f"small B={batch}")
    # a second launch at the same position reproduces the step bit for bit
    first = model.t["argmax_in"].tensor.clone()
    model.step()
    torch.cuda.synchronize()
    assert torch.equal(first, model.t["argmax_in"].tensor)


@pytest.mark.parametrize("batch", [1, 8])
def test_llama3_8b_dims_one_layer_elementwise(batch):
    """One layer at full Llama-3-8B dims: logits element-wise within rtol /
    atol 1e-2 of the oracle at batch 1; at batch 8 within it for all but
    0.1 % of the logits and within 2^-5 everywhere, the oracle's own noise
    floor for this layer (tests/test_oracle.py).  (From two layers on, +-1
    ulp of rounding noise in the activations alone moves some logits by
    more than that, so deeper stacks are bounded by magnitude and relative
    L2 instead.)"""
    cfg = LlamaConfig(num_layers=1)
    print(f"case llama3-8b dims, 1 layer, B={batch} kv=4096", flush=True)
    model = LlamaDecodeModel(cfg, batch=batch, kv_len=4096, seed=0)
    tokens = (np.arange(batch) * 15013 + 128000) % cfg.vocab
    model.set_input_tokens(tokens)
    model.step()
    torch.cuda.synchronize()
    rc, st = model.pk.status()
    assert rc == 0, st
    ref_logits, ref_ids = decode_step(cfg, batch, 4096, 64, 0, tokens)
    _check(model, tokens, ref_logits, ref_ids, f"llama3-8b 1 layer B={batch}", elementwise=True)


@pytest.mark.parametrize("batch", [1, 8])
def test_llama3_8b_dims_two_layers(batch):
    """Every op at its full Llama-3-8B shape (KV length 4096, vocab 128256):
    two layers keep rounding drift below the per-op tolerance."""
    cfg = LlamaConfig(num_layers=2)
    print(f"case llama3-8b dims, 2 layers, B={batch} kv=4096", flush=True)
    model = LlamaDecodeModel(cfg, batch=batch, kv_len=4096, seed=0)
    tokens = (np.arange(batch) * 15013 + 128000) % cfg.vocab
    model.set_input_tokens(tokens)
    model.step()
    torch.cuda.synchronize()
    rc, st = model.pk.status()
    assert rc == 0, st
    ref_logits, ref_ids = decode_step(cfg, batch, 4096, 64, 0, tokens)
    _check(model, tokens, ref_logits, ref_ids, f"llama3-8b 2 layers B={batch}")


@pytest.mark.parametrize("batch", [1, 8])
def test_llama3_8b_decode_step(batch):
    """The full 32-layer step.  Measured drift against the oracle grows with
    depth (relative L2 ~1e-5 at 2 layers, 3e-3 at 4, 8e-3 at 8, 2.5e-2 at
    32), so the 32-layer bound is 5e-2 relative L2 plus the exact token."""
    cfg = LlamaConfig()
    print(f"case llama3-8b B={batch} kv=4096", flush=True)
    model = LlamaDecodeModel(cfg, batch=batch, kv_len=4096, seed=0)
    tokens = (np.arange(batch) * 15013 + 128000) % cfg.vocab
    model.set_input_tokens(tokens)
    model.step()
    torch.cuda.synchronize()
    rc, st = model.pk.status()
    assert rc == 0, st
    ref_logits, ref_ids = decode_step(cfg, batch, 4096, 64, 0, tokens)
    _check(model, tokens, ref_logits, ref_ids, f"llama3-8b B={batch}", rel_l2=5e-2)
