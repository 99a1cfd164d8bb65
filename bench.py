"""Benchmark of the hip backend on one MI355X.

Headline (BASELINE.json metric): latency of one Llama-3-8B-shaped decode step
at batch 1 (32 layers, hidden 4096, GQA 32/8, head_dim 128, MLP 14336, vocab
128256, bf16 random-init weights, KV length 4096 in 64-token pages behind a
random page table), run as one persistent-megakernel launch per step.  The
fused operators of BASELINE configs 1-4 and the batch-8 step are reported in
the same JSON line under "fused_ops" / "decode_b8".

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-fused] [--no-cpu]

Prints exactly one JSON line on stdout.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
# HBM bytes per pk_worker_kernel launch of the batch-1 headline step, from
# rocprofv3 FETCH_SIZE / WRITE_SIZE (scaled by a 1 GiB copy kernel: x2.0 /
# x1.0), measured on the current kernel with ordinary launches (FETCH
# 7,650,294 KiB, WRITE 52,553 KiB per dispatch); the profile summary of the
# decode step has the runs.  The bytes a step moves do not depend on the task
# schedule.
PK_B1_TRAFFIC_BYTES = 15_721_272_310
MFMA_BF16_PEAK_TFS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s


def _events_time(torch, fn, iters: int) -> float:
    """Average milliseconds per call of fn (launches on torch's current stream)."""
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters


def _graph_time(torch, fn, per_graph: int = 20, replays: int = 5) -> float:
    """Average ms per call with launch overhead removed: `per_graph` calls are
    captured in one HIP graph and replayed."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=st):
            for _ in range(per_graph):
                fn()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    return _events_time(torch, g.replay, replays) / per_graph


def bench_fused(torch):
    import yirage_amd.fused as F

    dev = "cuda"
    gen = torch.Generator(device=dev).manual_seed(0)
    out = {}

    def rnd(shape, std, dtype):
        return (torch.randn(shape, generator=gen, device=dev) * std).to(dtype)

    # config 1: RMSNorm + linear, X[8,4096] f16, W[4096,4096] (K x N)
    x = rnd((8, 4096), 1.0, torch.float16)
    g = torch.ones(4096, dtype=torch.float16, device=dev)
    w = rnd((4096, 4096), 0.02, torch.float16)
    o = torch.empty((8, 4096), dtype=torch.float16, device=dev)
    ms = _graph_time(torch, lambda: F.rmsnorm_linear(x, g, w, eps=1e-6, out=o))
    b = 33_693_696
    out["rmsnorm_linear_b8"] = dict(us=ms * 1e3, gbs=b / ms / 1e6, frac_hbm=b / ms / 1e6 / HBM_PEAK_GBS)
    # config 2a / 2b: gated MLP W1, W3 [4096, 14336] bf16
    w1 = rnd((4096, 14336), 0.02, torch.bfloat16)
    w3 = rnd((4096, 14336), 0.02, torch.bfloat16)
    for B, b in ((8, 235_175_936), (128, 239_599_616)):
        xb = rnd((B, 4096), 1.0, torch.bfloat16)
        ob = torch.empty((B, 14336), dtype=torch.bfloat16, device=dev)
        ms = _graph_time(torch, lambda: F.gated_mlp(xb, w1, w3, out=ob), per_graph=10 if B > 8 else 20)
        flops = 4.0 * B * 4096 * 14336
        out[f"gated_mlp_b{B}"] = dict(us=ms * 1e3, gbs=b / ms / 1e6, frac_hbm=b / ms / 1e6 / HBM_PEAK_GBS,
                                      tflops=flops / ms / 1e9)
    del w1, w3
    # config 3: paged GQA decode, B=8, 32/8 heads, d=128, KV 4096 f16, 64-token pages
    B, Hq, Hkv, D, L, page = 8, 32, 8, 128, 4096, 64
    P = B * L // page
    kc = rnd((P, page, Hkv, D), 1.0, torch.float16)
    vc = rnd((P, page, Hkv, D), 1.0, torch.float16)
    idx = torch.randperm(P, generator=gen, device=dev).to(torch.int32)
    indptr = (torch.arange(B + 1, device=dev) * (L // page)).to(torch.int32)
    lens = torch.full((B,), L, dtype=torch.int32, device=dev)
    q = rnd((B, Hq, D), 1.0, torch.float16)
    oq = torch.empty_like(q)
    ms = _graph_time(torch, lambda: F.gqa_decode_paged(q, kc, vc, indptr, idx, lens, max_kv_len=L, out=oq))
    b = 2 * B * L * Hkv * D * 2 + 2 * B * Hq * D * 2 + (B + 1 + P) * 4
    out["gqa_decode_b8"] = dict(us=ms * 1e3, gbs=b / ms / 1e6, frac_hbm=b / ms / 1e6 / HBM_PEAK_GBS)
    del kc, vc
    # config 4: causal GQA prefill, S=2048, 32/8 heads, d=128 bf16
    S = 2048
    qq = rnd((1, S, 32, 128), 1.0, torch.bfloat16)
    kk = rnd((1, S, 8, 128), 1.0, torch.bfloat16)
    vv = rnd((1, S, 8, 128), 1.0, torch.bfloat16)
    oo = torch.empty_like(qq)
    ms = _graph_time(torch, lambda: F.gqa_prefill(qq, kk, vv, causal=True, out=oo), per_graph=10)
    flops = 4.0 * 128 * 32 * S * (S + 1) / 2
    out["gqa_prefill_s2048"] = dict(us=ms * 1e3, tflops=flops / ms / 1e9,
                                    frac_mfma=flops / ms / 1e9 / MFMA_BF16_PEAK_TFS)
    for v in out.values():
        for k in list(v):
            v[k] = round(v[k], 4)
    return out


def bench_mugraph_plans(torch) -> dict:
    """Device time (HIP-graph replay, launch overhead removed) of the saved
    muGraph candidates that run as generic steps or literally, tile by tile
    (customized ops no fused kernel covers): each distinct plan of the LoRA,
    qk-norm GQA, norm-transformer and MHA files (tests/golden/saved_mugraphs),
    one launch per operator against the same plan with its elementwise trees
    fused (fused elementwise launches), and against the plan whose customized
    ops each run as one tile-program launch (yr_hip_tb_program)."""
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests"))
    from yirage_amd import YirageHipError
    from yirage_amd import mugraph_json as MJ

    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "golden", "saved_mugraphs")
    files = [("single_lora.json", (1.0, 0.05, 0.05, 0.25)), ("qknorm_gqa_bs1_subset.json", (1.0, 0.02, 1.0)),
             ("ntrans_bs1.json", (1.0, 1.0, 1.0)), ("mha_bs1.json", (0.25, 0.25, 1.0))]
    out = {}
    for name, stds in files:
        gs = MJ.load(os.path.join(golden, name))
        seen = set()
        for i, g in enumerate(gs):
            try:
                p0 = g.plan(fuse=True, fuse_elementwise=False)
                p1 = g.plan(fuse=True)
                p2 = g.plan(fuse=True, tb_program=True)
            except YirageHipError:
                continue
            key = tuple(p0.describe())
            if key in seen:
                continue
            seen.add(key)
            gen = torch.Generator().manual_seed(i)
            ins = []
            for t, sd in zip(g.inputs, stds):
                n = sum((d - 1) * s_ for d, s_ in zip(t.dims, t.strides)) + 1
                base = (torch.randn(n, generator=gen) * sd).to(t.dtype.torch)
                ins.append(torch.as_strided(base, t.dims, t.strides).cuda())
            rec = {"steps": len(p0.steps)}
            for tag, p in (("one_launch_per_op", p0), ("elementwise_fused", p1), ("tile_program", p2)):
                if tag == "elementwise_fused" and p1.describe() == p0.describe():
                    continue
                if tag == "tile_program" and "tb_program" not in p2.describe():
                    continue
                ms = _graph_time(torch, lambda p=p: g._execute(p, ins, None), per_graph=10, replays=5)
                rec[tag] = dict(us=round(ms * 1e3, 2), launches=len(p.steps))
            out[f"{name}#{i}"] = rec
    return out


def _cpu_time(fn, warmup: int, reps: int) -> float:
    """Mean ms per call after `warmup` untimed calls (time.perf_counter), the
    method of the reference's CPU harness (benchmark/baselines/pytorch/
    rms_norm.py:30-53) with repetition counts sized to the op."""
    for _ in range(warmup):
        fn()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    return (time.perf_counter() - t0) / reps * 1e3


def cpu_fused(threads: int) -> dict:
    """The CPU oracle (oracle/yr_oracle.c: double accumulation, bf16 / f16
    rounding at the same tensor boundaries, OpenMP over `threads`) on the
    same shapes as BASELINE configs 1-4, seeded synthetic inputs."""
    import numpy as np

    from oracle import oracle as O

    rng = np.random.default_rng(0)
    out = {}

    def rec(name, ms, warmup, reps):
        out[name] = dict(cpu_ms=round(ms, 3), warmup=warmup, reps=reps, cores=threads)

    x = O.round_to(rng.standard_normal((8, 4096)), "f16")
    g = np.ones(4096, np.float32)
    w = O.synth((4096, 4096), "f16", 11, 0.02)
    rec("rmsnorm_linear_b8", _cpu_time(lambda: O.rmsnorm_linear(x, g, w, "f16", O.W_KN, 1e-6), 4, 32), 4, 32)
    w1 = O.synth((4096, 14336), "bf16", 12, 0.02)
    w3 = O.synth((4096, 14336), "bf16", 13, 0.02)
    xb = O.round_to(rng.standard_normal((8, 4096)), "bf16")
    rec("gated_mlp_b8", _cpu_time(lambda: O.gated_mlp(xb, w1, w3, "bf16"), 1, 4), 1, 4)
    xb = O.round_to(rng.standard_normal((128, 4096)), "bf16")
    rec("gated_mlp_b128", _cpu_time(lambda: O.gated_mlp(xb, w1, w3, "bf16"), 0, 1), 0, 1)
    del w1, w3
    B, Hq, Hkv, D, L, page = 8, 32, 8, 128, 4096, 64
    P = B * L // page
    kc = O.synth((P, page, Hkv, D), "f16", 14, 1.0)
    vc = O.synth((P, page, Hkv, D), "f16", 15, 1.0)
    idx = rng.permutation(P).astype(np.int32)
    indptr = (np.arange(B + 1) * (L // page)).astype(np.int32)
    lens = np.full(B, L, np.int32)
    q = O.to_float(O.synth((B, Hq, D), "f16", 16, 1.0), "f16")
    rec("gqa_decode_b8", _cpu_time(lambda: O.gqa_decode_paged(q, kc, vc, "f16", indptr, idx, lens), 1, 4), 1, 4)
    del kc, vc
    S = 2048
    qq = O.to_float(O.synth((1, S, 32, 128), "bf16", 17, 1.0), "bf16")
    kk = O.to_float(O.synth((1, S, 8, 128), "bf16", 18, 1.0), "bf16")
    vv = O.to_float(O.synth((1, S, 8, 128), "bf16", 19, 1.0), "bf16")
    rec("gqa_prefill_s2048", _cpu_time(lambda: O.gqa_prefill(qq, kk, vv, True), 0, 1), 0, 1)
    return out


def cpu_decode(batch: int, threads: int, sample_layers: int = 2, warmup: int = 1, reps: int = 2) -> dict:
    """The CPU oracle on a bounded sample of the same decode step:
    `sample_layers` full decoder layers (RMSNorm, QKV, RoPE + paged GQA at
    kv 4096 with the new token appended, O-proj + residual, RMSNorm, gate /
    up, SiLU-mul, down + residual), `warmup` untimed and `reps` timed passes
    each, scaled to 32 layers, plus the LM head and argmax (timed the same
    way).  Weight and cache generation are outside the timed region."""
    import numpy as np

    from oracle import oracle as O
    from yirage_amd.llama import LLAMA3_8B as cfg, page_table, rope_tables, tensor_seed, weight_shapes

    bf = "bf16"
    G, D, kv_len, page = cfg.num_q_heads // cfg.num_kv_heads, cfg.head_dim, 4096, 64
    indptr, indices, pool = page_table(batch, kv_len, page, 7)
    cos, sin = rope_tables(kv_len + 8, D, cfg.rope_theta)
    cos, sin = cos.float().numpy(), sin.float().numpy()
    qo = np.arange(batch + 1, dtype=np.int32)
    lpl = np.full(batch, kv_len % page, np.int32)
    ones = np.ones(cfg.hidden, np.float32)
    x0 = O.round_to(np.random.default_rng(0).standard_normal((batch, cfg.hidden)), bf)
    per_layer = []
    for layer in range(sample_layers):
        W = {n: O.synth(s, bf, tensor_seed(0, layer, n), 0.02) for n, s in weight_shapes(cfg).items()}
        rows = []
        for g in range(cfg.num_kv_heads):
            rows += [W["wq"][g * G * D:(g + 1) * G * D], W["wk"][g * D:(g + 1) * D], W["wv"][g * D:(g + 1) * D]]
        wqkv = np.ascontiguousarray(np.concatenate(rows, 0))
        kc = O.synth((pool, page, cfg.num_kv_heads, D), bf, tensor_seed(0, layer, "kc"), 1.0)
        vc = O.synth((pool, page, cfg.num_kv_heads, D), bf, tensor_seed(0, layer, "vc"), 1.0)

        def one_layer(x=x0):
            xn = O.round_to(O.rmsnorm(x, ones, cfg.eps), bf)
            qkv = O.round_to(O.linear(xn, wqkv, bf, O.W_NK), bf)
            att = O.round_to(O.paged_attention(qkv, cfg.num_q_heads, cfg.num_kv_heads, D, kc, vc, bf, qo, indptr,
                                               indices, lpl, cos, sin), bf)
            h = O.round_to(O.linear(att, W["wo"], bf, O.W_NK, residual=x), bf)
            hn = O.round_to(O.rmsnorm(h, ones, cfg.eps), bf)
            m = O.silu_mul(O.round_to(O.linear(hn, W["wg"], bf, O.W_NK), bf),
                           O.round_to(O.linear(hn, W["wu"], bf, O.W_NK), bf), bf)
            return O.round_to(O.linear(m, W["wd"], bf, O.W_NK, residual=h), bf)

        per_layer.append(_cpu_time(one_layer, warmup, reps))
        del W, kc, vc
    lm = O.synth((cfg.vocab, cfg.hidden), bf, tensor_seed(0, 0, "lm_head"), 0.02)
    t_lm = _cpu_time(lambda: O.argmax(O.round_to(O.linear(O.round_to(O.rmsnorm(x0, ones, cfg.eps), bf), lm, bf,
                                                                    O.W_NK), bf)), warmup, reps)
    step_ms = sum(per_layer) / sample_layers * cfg.num_layers + t_lm
    return dict(value=round(step_ms, 2), unit="ms", cores=threads, kind="port", warmup=warmup, reps=reps,
                sample=f"batch {batch}: {sample_layers} of 32 decoder layers ({warmup} untimed + {reps} timed "
                       f"passes each, mean scaled x32) + LM head/argmax ({warmup} + {reps}); kv 4096",
                layer_ms=[round(v, 2) for v in per_layer], lm_head_ms=round(t_lm, 2))


def _cpu_model() -> str:
    """The host CPU's model name (what lscpu prints as 'Model name')."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-fused", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-b8", action="store_true")
    ap.add_argument("--no-b16", action="store_true")
    ap.add_argument("--mugraph-plans", action="store_true",
                    help="only time the saved muGraph candidates' generic / literal plans (JSON line)")
    ap.add_argument("--no-coop", action="store_true",
                    help="ordinary (non-cooperative) launch of the persistent kernel, e.g. under rocprofv3")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only copy a 1 GiB device buffer 3 times (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the hip backend's persistent kernel runs on one "
              "GPU; a multi-GPU step would shard the weights column-/row-parallel per layer); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from yirage_amd.llama import LLAMA3_8B, LlamaDecodeModel

    torch.cuda.set_device(0)
    if args.mugraph_plans:
        print(json.dumps({"mugraph_plans": bench_mugraph_plans(torch)}))
        return
    if args.copy_calib:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        return
    model = LlamaDecodeModel(LLAMA3_8B, batch=1, kv_len=4096, seed=0)
    if args.no_coop:
        model.pk.set_cooperative(False)
    model.set_input_tokens([128000])
    for _ in range(args.warmup):
        model.step()
    torch.cuda.synchronize()
    rc, st = model.pk.status()
    if rc != 0:
        raise SystemExit(f"persistent kernel status {st}")
    ms = _events_time(torch, model.step, args.steps)
    rc, st = model.pk.status()
    if rc != 0:
        raise SystemExit(f"persistent kernel status {st}")
    # the same steps as passes of ONE launch (the reference's offline ypk()
    # runs a whole generation in one launch): no launch gap between steps
    ms_in = _events_time(torch, lambda: model.pk(max_iterations=args.steps), 1) / args.steps
    rc, st = model.pk.status()
    if rc != 0 or model.pk.iterations() != args.steps:
        raise SystemExit(f"persistent kernel status {st} after an in-launch run")
    step_bytes = model.weight_bytes() + model.kv_bytes()
    achieved = step_bytes / ms / 1e6
    info = model.pk.graph_info()
    # release device resources explicitly (not from __del__ at interpreter
    # shutdown, after a profiler may have torn down the runtime)
    model.pk.finalize()
    del model
    torch.cuda.empty_cache()

    extra = {}
    if not args.no_b8:
        m8 = LlamaDecodeModel(LLAMA3_8B, batch=8, kv_len=4096, seed=0)
        if args.no_coop:
            m8.pk.set_cooperative(False)
        m8.set_input_tokens([128000] * 8)
        for _ in range(max(1, args.warmup)):
            m8.step()
        ms8 = _events_time(torch, m8.step, max(5, args.steps // 2))
        b8 = m8.weight_bytes() + m8.kv_bytes()
        extra["decode_b8"] = dict(ms=round(ms8, 4), gbs=round(b8 / ms8 / 1e6, 1),
                                  frac_hbm=round(b8 / ms8 / 1e6 / HBM_PEAK_GBS, 4),
                                  tokens_per_s=round(8 / ms8 * 1e3, 1),
                                  weights="packed in stream order at compile (yr_pk_pack_weights)")
        m8.pk.finalize()
        del m8
        torch.cuda.empty_cache()
    if not args.no_b16:
        # 16 tokens per launch (the largest max_num_batched_tokens): 16
        # requests of one token each, 16-token MFMA tiles
        m16 = LlamaDecodeModel(LLAMA3_8B, batch=16, kv_len=4096, seed=0)
        if args.no_coop:
            m16.pk.set_cooperative(False)
        m16.set_input_tokens(list(range(128000, 128016)))
        for _ in range(max(1, args.warmup)):
            m16.step()
        ms16 = _events_time(torch, m16.step, max(5, args.steps // 2))
        b16 = m16.weight_bytes() + m16.kv_bytes()
        extra["decode_b16"] = dict(ms=round(ms16, 4), gbs=round(b16 / ms16 / 1e6, 1),
                                   frac_hbm=round(b16 / ms16 / 1e6 / HBM_PEAK_GBS, 4),
                                   tokens_per_s=round(16 / ms16 * 1e3, 1),
                                   weights="packed in stream order at compile (yr_pk_pack_weights)")
        m16.pk.finalize()
        del m16
        torch.cuda.empty_cache()
    if not args.no_fused:
        import yirage_amd.fused as F

        extra["fused_ops"] = bench_fused(torch)
        torch.cuda.synchronize()
        F._ws_cache.clear()
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O

        threads = os.cpu_count() or 1
        O.set_num_threads(threads)
        cpu = cpu_decode(1, threads)
        cpu.update(os_cpu_count=os.cpu_count(), torch_threads=torch.get_num_threads(), cpu_model=_cpu_model())
        if "decode_b8" in extra:
            extra["decode_b8"]["cpu_baseline"] = cpu_decode(8, threads)
        if "fused_ops" in extra:
            for k, v in cpu_fused(threads).items():
                extra["fused_ops"][k].update(v)

    line = {
        "metric": "fused-op latency (µs) & % HBM peak; 8B-shape decode step latency, batch 1",
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights ~N(0,0.02), KV cache ~N(0,1), seeded)",
        "config": {"workload": "llama3-8b-shape decode step, batch 1, kv 4096, persistent kernel",
                   "layers": 32, "hidden": 4096, "heads": "32/8", "head_dim": 128, "mlp": 14336,
                   "vocab": 128256, "page_size": 64, "parallelism": "single GPU",
                   "tasks_per_step": info["tasks"], "workers": info["workers"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": PK_B1_TRAFFIC_BYTES,
                     "algorithmic_bytes": step_bytes},
        "tokens_per_s": round(1e3 / ms, 2),
        "in_launch": {"ms_per_step": round(ms_in, 4), "steps_per_launch": args.steps,
                      "frac_hbm": round(step_bytes / ms_in / 1e6 / HBM_PEAK_GBS, 4)},
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
