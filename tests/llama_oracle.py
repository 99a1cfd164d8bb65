"""CPU oracle of the Llama-3-shaped decode step (test infrastructure).

Composes the oracle operators in the order of demo/llama3/demo.py:487-747,
rounding activations to bf16 at every inter-task tensor as the reference's
tasks do (rmsnorm.cuh:120-124, linear_cutlass.cuh epilogue, silu_mul.cuh:
31-40, multitoken_paged_attention_4_16.cuh).  Weights and the KV cache are
regenerated with the same counter-hash generator and seeds the device used.
"""
import numpy as np

from oracle import oracle as O
from yirage_amd.llama import QK_NORM_STD, page_table, rope_tables, tensor_seed, weight_shapes


def qk_norm_weights(cfg, seed, layer):
    """(q_norm, k_norm) float weights of a layer, as LlamaDecodeModel makes
    them (1 + N(0, QK_NORM_STD) rounded to bf16), or (None, None)."""
    if not cfg.qk_norm:
        return None, None
    return tuple(O.round_to(1.0 + O.to_float(O.synth((cfg.head_dim,), "bf16", tensor_seed(seed, layer, n),
                                                     QK_NORM_STD), "bf16"), "bf16") for n in ("qn", "kn"))


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
        qn, kn = qk_norm_weights(cfg, seed, layer)
        att = O.round_to(O.paged_attention(qkv, cfg.num_q_heads, cfg.num_kv_heads, D, kc, vc, bf, qo, indptr,
                                           indices, lpl, cos, sin, q_norm=qn, k_norm=kn), bf)
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


class ServingOracle:
    """Stateful oracle of the serving-mode model (LlamaDecodeModel with
    prompts): the same weights, its own paged KV caches (pool pages in the
    device layout), and one decode/extend step per call over the batch the
    device's metadata describes -- the composition of decode_step above with
    the multi-token paged attention (RoPE, cache append, causal mask over the
    new tokens) of multitoken_paged_attention_4_16.cuh:40-656."""

    def __init__(self, cfg, pool, page, seed, max_seq):
        bf = "bf16"
        self.cfg, self.page, self.seed = cfg, page, seed
        self.W = [{n: O.synth(shp, bf, tensor_seed(seed, layer, n), cfg.weight_std)
                   for n, shp in weight_shapes(cfg).items()} for layer in range(cfg.num_layers)]
        shp = (pool, page, cfg.num_kv_heads, cfg.head_dim)
        self.kc = [O.synth(shp, bf, tensor_seed(seed, layer, "kc"), 1.0) for layer in range(cfg.num_layers)]
        self.vc = [O.synth(shp, bf, tensor_seed(seed, layer, "vc"), 1.0) for layer in range(cfg.num_layers)]
        self.emb = O.synth((cfg.vocab, cfg.hidden), bf, tensor_seed(seed, 0, "embed"), cfg.weight_std)
        self.lm = O.synth((cfg.vocab, cfg.hidden), bf, tensor_seed(seed, 0, "lm_head"), cfg.weight_std)
        cos, sin = rope_tables(max(max_seq, 64), cfg.head_dim, cfg.rope_theta)
        self.cos, self.sin = cos.float().numpy(), sin.float().numpy()

    def step(self, tokens, qo_indptr, kv_indptr, kv_indices, last_page_len):
        """Logits [T, vocab] (bf16-rounded) and argmax ids of the T new tokens."""
        cfg, bf = self.cfg, "bf16"
        G, D = cfg.num_q_heads // cfg.num_kv_heads, cfg.head_dim
        x = O.to_float(self.emb[np.asarray(tokens, np.int64)], bf)
        ones = np.ones(cfg.hidden, np.float32)
        for layer in range(cfg.num_layers):
            W = self.W[layer]
            xn = O.round_to(O.rmsnorm(x, ones, cfg.eps), bf)
            rows = []
            for g in range(cfg.num_kv_heads):
                rows += [W["wq"][g * G * D:(g + 1) * G * D], W["wk"][g * D:(g + 1) * D], W["wv"][g * D:(g + 1) * D]]
            qkv = O.round_to(O.linear(xn, np.concatenate(rows, 0), bf, O.W_NK), bf)
            qn, kn = qk_norm_weights(cfg, self.seed, layer)
            att = O.round_to(O.paged_attention(qkv, cfg.num_q_heads, cfg.num_kv_heads, D, self.kc[layer],
                                               self.vc[layer], bf, qo_indptr, kv_indptr, kv_indices, last_page_len,
                                               self.cos, self.sin, q_norm=qn, k_norm=kn), bf)
            h = O.round_to(O.linear(att, W["wo"], bf, O.W_NK, residual=x), bf)
            hn = O.round_to(O.rmsnorm(h, ones, cfg.eps), bf)
            gate = O.round_to(O.linear(hn, W["wg"], bf, O.W_NK), bf)
            up = O.round_to(O.linear(hn, W["wu"], bf, O.W_NK), bf)
            x = O.round_to(O.linear(O.silu_mul(gate, up, bf), W["wd"], bf, O.W_NK, residual=h), bf)
        xn = O.round_to(O.rmsnorm(x, ones, cfg.eps), bf)
        logits = O.round_to(O.linear(xn, self.lm, bf, O.W_NK), bf)
        return logits, O.argmax(logits)
