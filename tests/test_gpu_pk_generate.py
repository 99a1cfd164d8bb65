"""GPU parity of a whole generation in ONE persistent-kernel launch.

The reference's offline ypk() runs every step of every request in one
launch: on EVENT_END_OF_TASK_GRAPH the device scheduler calls
prepare_next_batch and, while tokens remain, starts the next iteration
(include/yirage/persistent_kernel/persistent_kernel.cuh:841-857,
python/yirage/persistent_kernel.py:1322-1337, demo/llama3/demo.py:864-868).
Here one `pk()` call (max_iterations 0: until the batch is empty) must leave:

  * the device batch manager's final state -- request_ids, next_request_id,
    page_queue with its head / tail, step, tokens -- bit-identical to the
    CPU restatement (oracle.BatchManager) driven step by step with the
    tokens the device generated;
  * at every step of that replay, the argmax the oracle composition
    (tests/llama_oracle.ServingOracle) computes from the same inputs equal
    to the token the device kept, unless the oracle's top two logits are a
    near-tie (2^-7 relative, i.e. one bf16 ulp; reported);
  * the paged K / V caches of every layer at every position the replay
    wrote within rtol/atol 1e-2 of the oracle's in layer 0 (identical
    inputs) and 2e-2 * max(1, max|v|) deeper (rounding noise of the layers
    below);
  * the number of passes the device ran equal to the replay's steps + 1
    (the first pass runs an empty batch and schedules the first one).

Then a second launch with max_iterations 1 (an empty batch) must leave
the state as it is, and re-initialising the batch and generating again must
give identical tokens (the event epochs fast-forwarded after the early stop
are consistent).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.llama_oracle import ServingOracle
from tests.test_gpu_pk_serving import CFG, _simulate_first_output
from yirage_amd.llama import LlamaDecodeModel

pytestmark = pytest.mark.gpu


def _replay(model, prompts, MR, MT, pool, page, max_seq, seed, eos, dev_tokens):
    """Drive the CPU batch manager and the oracle model with the device's
    kept tokens; returns (batch manager, oracle, steps, near-ties)."""
    tokens = np.zeros((len(prompts), max_seq), np.int64)
    for i, p in enumerate(prompts):
        tokens[i, :len(p)] = p
    bm = O.BatchManager(MR, MT, pool, page, tokens, np.array([len(p) for p in prompts], np.int32), eos)
    orc = ServingOracle(CFG, pool, page, seed, max_seq)
    more = bm.prepare_next()
    steps = near = 0
    while more:
        T = int(bm["qo_indptr"][MR])
        logits, ids = orc.step(bm["input_tokens"][:T], bm["qo_indptr"], bm["kv_indptr"], bm["kv_indices"],
                               bm["last_page_len"])
        out = ids.copy()
        for s in range(MR):
            rid = int(bm["request_ids"][s])
            if rid < 0:
                continue
            step, plen = int(bm["step"][rid]), len(prompts[rid])
            for j in range(int(bm["qo_indptr"][s]), int(bm["qo_indptr"][s + 1])):
                pos = step + (j - int(bm["qo_indptr"][s])) + 1
                if pos >= plen and pos < max_seq:
                    kept = int(dev_tokens[rid, pos])
                    if kept != int(ids[j]):
                        top = np.sort(logits[j])[-2:]
                        assert top[1] - top[0] <= 2 ** -7 * max(abs(top[1]), 1e-3), \
                            f"step {steps}: request {rid} position {pos}: device {kept} oracle {ids[j]}"
                        near += 1
                    out[j] = kept
        bm["output_tokens"][:T] = out
        more = bm.prepare_next()
        steps += 1
        assert steps < 1000
    return bm, orc, steps, near


def _check_caches(model, orc):
    """Whole caches: both started from the same synthetic values, so slots
    nobody wrote compare equal and every appended slot is checked."""
    for layer in range(CFG.num_layers):
        for name, dc, oc in (("k", model.kc[layer], orc.kc[layer]), ("v", model.vc[layer], orc.vc[layer])):
            a_ = dc.float().cpu().numpy()
            b_ = O.to_float(oc, "bf16").reshape(a_.shape)
            e_ = np.abs(a_ - b_)
            if layer == 0:
                bad = e_ > 1e-2 + 1e-2 * np.abs(b_)
            else:
                bad = e_ > 2e-2 * np.maximum(1.0, np.abs(b_).max(-1, keepdims=True))
            assert not bad.any(), f"cached {name} layer {layer}: {bad.sum()} values differ, max diff {e_.max()}"


@pytest.mark.parametrize("MR,MT,lens", [(3, 8, (9, 70, 3, 20))])
def test_generation_in_one_launch(MR, MT, lens):
    page, max_seq = 64, 80
    npg = (max_seq + page - 1) // page
    pool = MR * npg
    print(f"case generate MR={MR} MT={MT} prompts {list(lens)}", flush=True)
    for seed in range(5, 25):
        rng = np.random.default_rng(seed)
        prompts = [rng.integers(0, CFG.vocab, n).tolist() for n in lens]
        eos, gap = _simulate_first_output(prompts, MR, MT, pool, page, max_seq, seed, 1)
        if gap > 0.1:
            break
    print(f"  seed {seed} eos token {eos} (logit gap {gap:.3f})", flush=True)
    model = LlamaDecodeModel(CFG, batch=MR, page_size=page, seed=seed, with_prepare=True, prompts=prompts,
                             max_tokens=MT, max_requests=MR, max_seq=max_seq, eos_token_id=eos)
    torch.cuda.synchronize()
    passes = model.generate(0)
    torch.cuda.synchronize()
    rc, st = model.pk.status()
    assert rc == 0, f"status {st}"
    dev_tokens = model.meta["tokens"].cpu().numpy().copy()
    dev_step = model.meta["step"].cpu().numpy().copy()
    state = model.pk.batch_state()
    print(f"  one launch ran {passes} passes; steps {dev_step.tolist()}", flush=True)

    bm, orc, steps, near = _replay(model, prompts, MR, MT, pool, page, max_seq, seed, eos, dev_tokens)
    print(f"  replay: {steps} steps, {near} near-ties", flush=True)
    assert passes == steps + 1
    assert np.array_equal(dev_tokens, bm["tokens"]), "tokens differ"
    assert np.array_equal(dev_step, bm["step"]), "step differs"
    for k in ("request_ids", "next_request_id", "page_queue", "page_queue_head", "page_queue_tail"):
        assert np.array_equal(state[k], bm[k]), f"{k}: device {state[k].tolist()} oracle {bm[k].tolist()}"
    assert bm["next_request_id"][0] == len(prompts) and (bm["request_ids"] == -1).all()
    assert bm["step"][1] == lens[1] and bm["tokens"][1, lens[1]] == eos  # request 1 ended on EOS
    _check_caches(model, orc)

    # an empty batch: one more pass changes nothing but runs cleanly
    model.pk(max_iterations=1)
    torch.cuda.synchronize()
    assert model.pk.status()[0] == 0
    assert model.pk.iterations() == 1
    assert np.array_equal(model.meta["tokens"].cpu().numpy(), dev_tokens)

    # the same requests again from a fresh batch state: identical tokens
    model.meta["step"].zero_()
    model.meta["tokens"].copy_(torch.from_numpy(np.where(np.arange(max_seq)[None, :] < np.array(lens)[:, None],
                                                         dev_tokens, 0)))
    model.pk.init_batch()
    passes2 = model.generate(0)
    torch.cuda.synchronize()
    assert model.pk.status()[0] == 0
    assert passes2 == passes
    assert np.array_equal(model.meta["tokens"].cpu().numpy(), dev_tokens), "second generation differs"
