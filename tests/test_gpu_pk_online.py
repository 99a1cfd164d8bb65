"""GPU parity of the persistent kernel in online mode
(persistent_kernel.cuh:325-351): one request whose host feeds, per launch,
how many tokens it accepted (meta tensor num_new_tokens, the reference's
new_token_nums).  The device's prepare_batch advances step[0] by it and
reports whether the sequence continues (not at max length, the token after
the old step not eos); both must equal the CPU restatement
(oracle.BatchManager.prepare_online), and the decode step itself the oracle
composition, launch after launch."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.llama_oracle import decode_step
from yirage_amd.llama import LlamaConfig, LlamaDecodeModel

pytestmark = pytest.mark.gpu


def test_online_mode_step_advance_and_stop():
    cfg = LlamaConfig(num_layers=2, hidden=1024, num_q_heads=8, num_kv_heads=2, head_dim=128, intermediate=2048,
                      vocab=4096)
    kv_len, eos = 100, 17
    print("case online mode, 2 layers, B=1 kv=100", flush=True)
    model = LlamaDecodeModel(cfg, batch=1, kv_len=kv_len, seed=3, with_prepare=True, eos_token_id=eos,
                             mode="online")
    meta = model.meta
    msl = model.max_seq
    tokens = np.zeros((1, msl), np.int64)
    bm = O.BatchManager(1, 1, model.max_pages, 64, tokens, np.int32([kv_len]), eos)
    # (accepted tokens, token written after the old step) per launch; the last one is eos
    plan = [(1, 5), (2, 9), (1, eos)]
    step = kv_len - 1
    meta["step"][0] = step
    bm["step"][0] = step
    for i, (n, nxt) in enumerate(plan):
        meta["num_new_tokens"][0] = n
        meta["tokens"][0, step + 1] = nxt
        bm["tokens"][0, step + 1] = nxt
        model.set_input_tokens([1234 + i])
        model.pk(max_iterations=1)
        torch.cuda.synchronize()
        rc, st = model.pk.status()
        assert rc == 0, st
        more = bm.prepare_online([n])
        assert int(meta["step"][0]) == int(bm["step"][0]) == step + n, f"launch {i}: step"
        assert bool(st[1]) == more == (nxt != eos), f"launch {i}: continue flag {st[1]}"
        step += n
    # the step itself (first launch's inputs) against the oracle composition
    model2 = LlamaDecodeModel(cfg, batch=1, kv_len=kv_len, seed=3, with_prepare=True, eos_token_id=eos,
                              mode="online")
    model2.set_input_tokens([1234])
    model2.pk(max_iterations=1)
    torch.cuda.synchronize()
    ref_logits, ref_ids = decode_step(cfg, 1, kv_len, 64, 3, np.array([1234]))
    got = model2.t["argmax_in"].tensor
    if model2.t["argmax_in"].ll:
        rows, cols = model2.t["argmax_in"].dims
        got = got.view(rows, cols // 2, 4)[..., :2].reshape(rows, cols)
    got = got.float().cpu().numpy()[:1]
    err = np.abs(got - ref_logits)
    print(f"  logits max abs err {err.max():.4f}", flush=True)
    assert err.max() <= 2e-2 * max(1.0, float(np.abs(ref_logits).max()))
