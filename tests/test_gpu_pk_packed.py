"""Packed linear weights (batch > 1 graphs).

`compile()` of a graph with max_num_batched_tokens > 1 gives every linear
task a copy of its weights in the order the task streams them (16-row x
32-column MFMA fragments, 1 KiB per load instruction; yr_pk_pack_weights).
The task reads the same values in the same order either way, so logits and
tokens must be bit-identical with and without the copy, for 8- and 16-token
tiles, for tasks that straddle two weight segments (QKV) and for the
[gate | up] pairs; the copy's size is checked against the linear tasks'
padded rows.  The oracle parity of the packed path is covered by every
batch > 1 decode / serving test, which now runs packed.
"""
import numpy as np
import pytest
import torch

from yirage_amd.llama import LlamaConfig, LlamaDecodeModel

pytestmark = pytest.mark.gpu

CFG = LlamaConfig(num_layers=2, hidden=1024, num_q_heads=8, num_kv_heads=2, intermediate=2048, vocab=4096)


@pytest.mark.parametrize("batch", [3, 8, 13, 16])
def test_packed_weights_bit_identical(batch):
    print(f"case packed weights batch {batch}", flush=True)
    model = LlamaDecodeModel(CFG, batch=batch, kv_len=100, seed=4)
    model.set_input_tokens(np.arange(batch) * 257 % CFG.vocab)

    def step():
        model.step()
        torch.cuda.synchronize()
        assert model.pk.status()[0] == 0
        return model.t["argmax_in"].tensor[:batch].clone(), model.meta["output_tokens"][:batch].clone()

    packed_logits, packed_tok = step()  # compile() packed them
    assert model.pk.pack_weights(False) == 0
    plain_logits, plain_tok = step()
    assert torch.equal(packed_logits, plain_logits), "packed and plain weights give different logits"
    assert torch.equal(packed_tok, plain_tok)
    nbytes = model.pk.pack_weights(True)
    # every linear task's rows rounded up to 16-row tiles (small tasks of
    # this toy model: up to 3x), all of K (bf16); the padding is never read
    H, I, V = CFG.hidden, CFG.intermediate, CFG.vocab
    lin = CFG.num_layers * ((CFG.num_q_heads + 2 * CFG.num_kv_heads) * CFG.head_dim * H + H * H + 2 * I * H + H * I)
    assert lin + V * H <= nbytes // 2 <= 3 * (lin + V * H), nbytes
    again_logits, again_tok = step()
    assert torch.equal(again_logits, plain_logits)
    assert torch.equal(again_tok, plain_tok)
    model.pk.finalize()


def test_batch1_packs_nothing():
    model = LlamaDecodeModel(CFG, batch=1, kv_len=100, seed=4)
    assert model.pk.pack_weights(True) == 0
    model.pk.finalize()
