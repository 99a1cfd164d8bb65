"""The persistent kernel's watchdog, forced from the host.

Every wait of the worker kernel (event polls, link-word and split-record
re-reads, the grid barrier between passes) is bounded by a spin limit; on
expiry the kernel sets status[0], records where it gave up in status[2] and
drains: every later wait sees the flag and gives up at once, so all waves
exit.  The reference's kernel has no such bound (a lost dependency spins
forever, persistent_kernel.cuh:454-727); this is the hip backend's failure
path, not a parity item.

With a spin limit of 1 poll the step's first dependency that is not already
there fires the watchdog.  The test checks that

  * the launch returns (the grid drains; pytest's per-test timeout would
    name a hang),
  * status() reports the timeout (rc YR_E_TIMEOUT, status[0] == 1),
  * after reset_status() and the default limit restored, the same step on
    the same inputs gives bit-identical logits and tokens to a step run
    before the timeout (the counters, tickets and tagged words were re-based
    consistently).

Batch 1 exercises the link-tensor paths (tag re-reads), batch 3 the event
paths.
"""
import numpy as np
import pytest
import torch

from tests.test_gpu_task_graph import _values
from yirage_amd.llama import LlamaConfig, LlamaDecodeModel

pytestmark = pytest.mark.gpu

CFG = LlamaConfig(num_layers=2, hidden=1024, num_q_heads=8, num_kv_heads=2, intermediate=2048, vocab=4096)
YR_E_TIMEOUT = -6


@pytest.mark.parametrize("batch", [1, 3])
def test_watchdog_fires_drains_and_recovers(batch):
    print(f"case watchdog batch {batch}", flush=True)
    model = LlamaDecodeModel(CFG, batch=batch, kv_len=130, seed=9)
    model.set_input_tokens([11, 2222, 3333][:batch])
    kc0 = [k.clone() for k in model.kc]
    vc0 = [v.clone() for v in model.vc]

    def restore():
        for i in range(CFG.num_layers):
            model.kc[i].copy_(kc0[i])
            model.vc[i].copy_(vc0[i])
        model.meta["output_tokens"].zero_()

    model.step()
    torch.cuda.synchronize()
    assert model.pk.status()[0] == 0
    want = _values(model.t["argmax_in"])[:batch].clone()
    want_tok = model.meta["output_tokens"].clone()

    restore()
    model.pk.set_spin_limit(1)
    model.step()
    torch.cuda.synchronize()  # the grid drained
    rc, st = model.pk.status()
    print(f"  after the forced timeout: rc {rc} status {st}", flush=True)
    assert rc == YR_E_TIMEOUT and st[0] == 1

    model.pk.set_spin_limit(1 << 26)
    model.pk.reset_status()
    assert model.pk.status() == (0, [0, 0, 0, 0])
    restore()
    model.step()
    torch.cuda.synchronize()
    assert model.pk.status()[0] == 0
    got = _values(model.t["argmax_in"])[:batch]
    assert torch.equal(got, want), "logits after recovery differ"
    assert torch.equal(model.meta["output_tokens"], want_tok)
    model.pk.finalize()


def test_watchdog_in_a_whole_generation_launch():
    """A multi-pass launch (a serving graph run until the batch is empty)
    whose first dependency wait gives up: the workers still inside the pass
    leave it, the rest give up at the grid barrier, the launch returns with
    YR_E_TIMEOUT; after reset_status, init_batch and restored caches the
    same generation gives the tokens a clean run gave."""
    from tests.test_gpu_pk_serving import CFG as SCFG
    MR, MT, page, max_seq = 3, 8, 64, 40
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, SCFG.vocab, n).tolist() for n in (9, 17, 3, 12)]
    print("case watchdog whole-generation launch", flush=True)
    model = LlamaDecodeModel(SCFG, batch=MR, page_size=page, seed=5, with_prepare=True, prompts=prompts,
                             max_tokens=MT, max_requests=MR, max_seq=max_seq, eos_token_id=-1)
    tokens0 = model.meta["tokens"].clone()
    kc0 = [k.clone() for k in model.kc]
    vc0 = [v.clone() for v in model.vc]

    def restore():
        model.meta["step"].zero_()
        model.meta["tokens"].copy_(tokens0)
        for i in range(SCFG.num_layers):
            model.kc[i].copy_(kc0[i])
            model.vc[i].copy_(vc0[i])
        model.pk.init_batch()

    passes = model.generate(0)
    torch.cuda.synchronize()
    assert model.pk.status()[0] == 0
    want = model.meta["tokens"].clone()

    restore()
    model.pk.set_spin_limit(1)
    model.pk(max_iterations=0)
    torch.cuda.synchronize()  # every worker left the launch
    rc, st = model.pk.status()
    print(f"  after the forced timeout: rc {rc} status {st}", flush=True)
    assert rc == YR_E_TIMEOUT and st[0] == 1

    model.pk.set_spin_limit(1 << 26)
    model.pk.reset_status()
    restore()
    assert model.generate(0) == passes
    torch.cuda.synchronize()
    assert model.pk.status()[0] == 0
    assert torch.equal(model.meta["tokens"], want), "generation after recovery differs"
    model.pk.finalize()
