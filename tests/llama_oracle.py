"""CPU oracle of the Llama-3-shaped decode step (test infrastructure).

Composes the oracle operators in the order of demo/llama3/demo.py:487-747,
rounding activations to bf16 at every inter-task tensor as the reference's
tasks do (rmsnorm.cuh:120-124, linear_cutlass.cuh epilogue, silu_mul.cuh:
31-40, multitoken_paged_attention_4_16.cuh).  Weights and the KV cache are
regenerated with the same counter-hash generator and seeds the device used.
"""
import numpy as np

from oracle import oracle as O
from yirage_amd.llama import page_table, rope_tables, tensor_seed, weight_shapes


def decode_step(cfg, batch, kv_len, page, seed, tokens, return_logits=True):
    bf = "bf16"
    G = cfg.num_q_heads // cfg.num_kv_heads
    D = cfg.head_dim
    indptr, indices, pool = page_table(batch, kv_len, page, seed + 7)
    cos, sin = rope_tables(max(kv_len + 8, 64), D, cfg.rope_theta)
    cos = cos.float().numpy()
    sin = sin.float().numpy()
    qo = np.arange(batch + 1, dtype=np.int32)
    lpl = np.full(batch, kv_len % page, np.int32)
    emb = O.synth((cfg.vocab, cfg.hidden), bf, tensor_seed(seed, 0, "embed"), cfg.weight_std)
    x = O.to_float(emb[np.asarray(tokens, np.int64)], bf)
    del emb
    ones = np.ones(cfg.hidden, np.float32)
    for layer in range(cfg.num_layers):
        W = {n: O.synth(shp, bf, tensor_seed(seed, layer, n), cfg.weight_std) for n, shp in weight_shapes(cfg).items()}
        xn = O.round_to(O.rmsnorm(x, ones, cfg.eps), bf)
        # QKV in the per-kv-group shuffled order [q(G heads) | k | v] x Hkv
        rows = []
        for g in range(cfg.num_kv_heads):
            rows.append(W["wq"][g * G * D:(g + 1) * G * D])
            rows.append(W["wk"][g * D:(g + 1) * D])
            rows.append(W["wv"][g * D:(g + 1) * D])
        wqkv = np.concatenate(rows, 0)
        qkv = O.round_to(O.linear(xn, wqkv, bf, O.W_NK), bf)
        shp = (pool, page, cfg.num_kv_heads, D)
        kc = O.synth(shp, bf, tensor_seed(seed, layer, "kc"), 1.0)
        vc = O.synth(shp, bf, tensor_seed(seed, layer, "vc"), 1.0)
        att = O.round_to(O.paged_attention(qkv, cfg.num_q_heads, cfg.num_kv_heads, D, kc, vc, bf, qo, indptr,
                                           indices, lpl, cos, sin), bf)
        h = O.round_to(O.linear(att, W["wo"], bf, O.W_NK, residual=x), bf)
        hn = O.round_to(O.rmsnorm(h, ones, cfg.eps), bf)
        gate = O.round_to(O.linear(hn, W["wg"], bf, O.W_NK), bf)
        up = O.round_to(O.linear(hn, W["wu"], bf, O.W_NK), bf)
        m = O.silu_mul(gate, up, bf)
        x = O.round_to(O.linear(m, W["wd"], bf, O.W_NK, residual=h), bf)
        del W
    xn = O.round_to(O.rmsnorm(x, ones, cfg.eps), bf)
    lm = O.synth((cfg.vocab, cfg.hidden), bf, tensor_seed(seed, 0, "lm_head"), cfg.weight_std)
    logits = O.round_to(O.linear(xn, lm, bf, O.W_NK), bf)
    return logits, O.argmax(logits)
