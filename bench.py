#!/usr/bin/env python3
"""Benchmark of the Qwen3 forward hot path on one MI355X.

Workload (headline): Qwen3-0.6B architecture, random-init fp16 weights N(0, 0.02) (seed 1), batch 1. A 32-token
prompt is prefilled (untimed), then W warmup and K timed greedy decode steps run with the sampled token fed back on
the device. A "step" is one decode token. Also measured in the same run:
  * prefill of a 2048-token prompt (tok/s, and its algorithmic FLOP/s against the 2.5 PFLOP/s dense fp16 peak in
    "prefill_roofline"), on the fp16 model and with its projections group-quantized (int8, int4),
  * the dominant decode kernel: k_decode_xcd (one launch = one whole token, every layer split over the 8 XCDs) or
    k_decode_persistent when the device runs that one, timed with HIP events on the stream it is launched on; the
    fused RMSNorm + QKV GEMV
    (4096 x 1024 fp16, over weight copies larger than the 256 MB Infinity Cache) is reported beside it,
  * every decode projection shape (q, k/v, o, gate/up, down, LM head) as an fp16 GEMV at batch 1 and as the
    int8 / int4 group-quantized matmul (group 64, fp16 scales) at batch 1 and 8, in GB/s against 8 TB/s,
  * the Qwen3-4B ragged decode batch (16 sequences, seeded KV lengths in [64, 4096]),
  * Qwen3-4B greedy decode at batch 1 (per-op kernels replayed as a HIP graph),
  * the kept C++ host API (GenerationContext::Generate through soc_amd/apps/soc_generate, a child process) on the
    headline workload, wall clock,
  * the reference CPU runtime on this host for every configuration (config 1 in full on the compiled reference, one
    core; configs 4 and 5 extrapolated from one layer on the bit-identical restatement, all host threads).
HBM traffic per launch of the dominant kernel comes from the rocprofv3 FETCH_SIZE / WRITE_SIZE summary in
profiles/ (scaled by the same counters over a plain copy of known size), when that summary exists.
Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import soc_amd as S  # noqa: E402

HBM_PEAK_GBS = 8000.0
PROMPT = 32


def decode_bytes_per_token(cfg: S.QwenConfig, kv_len: float) -> float:
    """Algorithmic HBM bytes of one decode token: every weight once (tied head once), gains, one embedding row,
    and the fp16 KV read of kv_len positions plus the write of one (28 x 2 x 8 x 128 x 2 B per position)."""
    H, I, L = cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers
    per_layer = (cfg.q_dim + 2 * cfg.kv_dim) * H + H * cfg.q_dim + 3 * I * H
    weights = 2 * (L * per_layer + cfg.vocab_size * H)
    gains = 2 * (L * (2 * H + 2 * cfg.head_dim) + H)
    embed_row = 2 * H
    kv_pos = L * 2 * cfg.num_key_value_heads * cfg.head_dim * 2
    return weights + gains + embed_row + kv_pos * (kv_len + 1)


def bench_decode(ctx, m, cfg, steps: int, warmup: int):
    cap = PROMPT + warmup + steps + 8
    kv = S.KVCache(m, 1, cap)
    prompt = S.synth_tokens(1, "prompt", cfg.vocab_size, PROMPT)
    _, tok = S.prefill(m, kv, 0, prompt)
    if warmup:
        toks = S.decode_steps(m, kv, 0, tok, warmup)
        tok = int(toks[-1])
    start_len = kv.length(0)
    ctx.synchronize()
    ctx.timer_start()
    toks = S.decode_steps(m, kv, 0, tok, steps)
    ms = ctx.timer_stop()
    ctx.synchronize()
    mean_kv = start_len + (steps - 1) / 2.0
    kv.close()
    return ms, mean_kv, toks


FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA


def prefill_flop(cfg, n: int) -> float:
    """Algorithmic FLOP of an n-token prefill: the projections (2 per weight per row), causal attention (q.k and p.v
    over the keys each row sees: 4 d flops per (head, row, visible key)) and the last row's LM head."""
    H, I, d = cfg.hidden_size, cfg.intermediate_size, 128
    qd, kvd = cfg.num_attention_heads * d, cfg.num_key_value_heads * d
    proj = 2.0 * n * (H * (qd + 2 * kvd) + qd * H + 2 * H * I + I * H)
    attn = 4.0 * d * cfg.num_attention_heads * n * (n + 1) / 2
    return cfg.num_hidden_layers * (proj + attn) + 2.0 * H * cfg.vocab_size


def bench_prefill(ctx, m, cfg, n: int = 2048):
    kv = S.KVCache(m, 1, n + 8)
    ids = S.synth_tokens(4, "prefill", cfg.vocab_size, n)
    S.prefill(m, kv, 0, ids[:64])  # warm the prefill path and its scratch
    kv.reset(0)
    S.prefill(m, kv, 0, ids)
    kv.reset(0)
    ctx.synchronize()
    ctx.timer_start()
    S.prefill(m, kv, 0, ids)
    ms = ctx.timer_stop()
    kv.close()
    return ms


def bench_prefill_quant(ctx, cfg, n: int = 2048):
    """Prefill of n tokens on the same model with its projections group-quantized (int8, int4): each layer's codes
    dequantized to fp16, then the fp16 prefill kernels."""
    out = {"workload": f"Qwen3-0.6B seed-1 weights, projections group-64 quantized, {n}-token prompt"}
    for bits in (8, 4):
        m = S.Model(ctx, cfg).synthesize(1, 0.02).quantize(bits)
        try:
            ms = bench_prefill(ctx, m, cfg, n)
        finally:
            m.close()
        out[f"int{bits}_ms"] = round(ms, 3)
        out[f"int{bits}_tok_s"] = round(n / (ms * 1e-3), 1)
    return out


def bench_decode_4b(ctx, steps: int = 64, warmup: int = 8):
    """Qwen3-4B greedy decode at batch 1 (seed-1 N(0, 0.02) weights) after the same 32-token prompt: the per-op
    kernels of one token replayed as a HIP graph (the one-launch kernel covers Qwen3-0.6B only)."""
    cfg = S.QWEN3_4B
    m = S.Model(ctx, cfg).synthesize(1, 0.02)
    try:
        ms, mean_kv, _ = bench_decode(ctx, m, cfg, steps, warmup)
        path = m.decode_path()
    finally:
        m.close()
    per_tok = ms / steps
    bpt = decode_bytes_per_token(cfg, mean_kv)
    gbs = bpt / (per_tok * 1e-3) / 1e9
    return {"workload": "Qwen3-4B greedy decode, batch 1, 32-token prompt", "decode_path": path, "steps": steps,
            "ms_per_token": round(per_tok, 4), "tok_s": round(1000.0 / per_tok, 1), "bytes_per_token": int(bpt),
            "hbm_gbs": round(gbs, 1), "hbm_roofline_frac": round(gbs / HBM_PEAK_GBS, 4)}


RAGGED_SEQS, RAGGED_STEPS, RAGGED_MIN, RAGGED_MAX = 16, 64, 64, 4096


def ragged_bytes_per_step(cfg: S.QwenConfig, kv_lens) -> float:
    """Algorithmic HBM bytes of one ragged step: every weight once (tied head once), gains, one embedding row per
    sequence, and each sequence's fp16 KV read of S_i positions plus the write of one."""
    H, I, L = cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers
    per_layer = (cfg.q_dim + 2 * cfg.kv_dim) * H + H * cfg.q_dim + 3 * I * H
    weights = 2 * (L * per_layer + cfg.vocab_size * H)
    gains = 2 * (L * (2 * H + 2 * cfg.head_dim) + H)
    kv_pos = L * 2 * cfg.num_key_value_heads * cfg.head_dim * 2
    return weights + gains + len(kv_lens) * 2 * H + kv_pos * float(sum(s + 1 for s in kv_lens))


def bench_ragged(ctx, steps: int = 64):
    """Qwen3-4B ragged continuous-batch decode: 16 sequences with seeded KV lengths U[64, 4096] (seeded N(0,1) fp16
    cache contents), 64 greedy steps of one token per sequence, each step one replay of the captured batch step."""
    cfg = S.QWEN3_4B
    m = S.Model(ctx, cfg).synthesize(1, 0.02)
    lens = S.synth_int_uniform(5, "ragged.kv_len", RAGGED_MIN, RAGGED_MAX, RAGGED_SEQS).astype(np.int64)
    kv = S.KVCache(m, RAGGED_SEQS, RAGGED_MAX + 2 * RAGGED_STEPS + 8)
    try:
        for slot, n in enumerate(lens):
            kv.fill_synthetic(slot, int(n), 7)
        slots = np.arange(RAGGED_SEQS, dtype=np.int32)
        toks = S.synth_tokens(6, "ragged.tokens", cfg.vocab_size, RAGGED_SEQS)
        warm = S.decode_batch_steps(m, kv, slots, toks, steps)  # builds and replays the step graph
        start = [kv.length(int(i)) for i in slots]
        ctx.synchronize()
        ctx.timer_start()
        out = S.decode_batch_steps(m, kv, slots, warm[-1], steps)
        ms = ctx.timer_stop()
    finally:
        kv.close()
        m.close()
    per_step = ms / steps
    mean_bytes = np.mean([ragged_bytes_per_step(cfg, [s + t for s in start]) for t in range(steps)])
    gbs = mean_bytes / (per_step * 1e-3) / 1e9
    return {"workload": "Qwen3-4B ragged decode, 16 sequences, KV lengths U[64,4096] (seed 5), 64 steps",
            "kv_lengths": [int(x) for x in lens], "tok_s": round(RAGGED_SEQS * steps / (ms * 1e-3), 1),
            "ms_per_step": round(per_step, 4), "bytes_per_step": int(mean_bytes), "hbm_gbs": round(gbs, 1),
            "hbm_roofline_frac": round(gbs / HBM_PEAK_GBS, 4), "tokens_head": [int(t) for t in out[0][:4]]}


def bench_gemv_kernel(ctx, n=4096, k=1024, iters=200):
    """Average duration of the decode GEMV kernel over weight copies that defeat the Infinity Cache."""
    wbytes = n * k * 2
    copies = max(2, (640 << 20) // wbytes)
    dw = ctx.alloc(wbytes * copies)
    dx = ctx.upload(S.synth_normal_f16(5, "bench.x", 1.0, k))
    dy = ctx.alloc(n * 4)
    try:
        for i in range(4):
            S.gemv_f16(ctx, dw + (i % copies) * wbytes, dx, dy, n, k)
        ctx.synchronize()
        ctx.timer_start()
        for i in range(iters):
            S.gemv_f16(ctx, dw + (i % copies) * wbytes, dx, dy, n, k)
        ms = ctx.timer_stop()
    finally:
        for p in (dw, dx, dy):
            ctx.free(p)
    us = ms * 1e3 / iters
    alg_bytes = 2 * n * k + 2 * k + 4 * n
    return us, alg_bytes


# Decode projection shapes of Qwen3-0.6B (out x in): the GEMV and group-quantized matmul microbenchmarks
OP_SHAPES = [("q_proj", 2048, 1024), ("k_proj/v_proj", 1024, 1024), ("o_proj", 1024, 2048),
             ("gate/up_proj", 3072, 1024), ("down_proj", 1024, 3072), ("lm_head", 151936, 1024)]


def _timed_op(ctx, launch, copies: int, iters: int) -> float:
    """Average microseconds of `launch(i)` (i selects the weight copy) over `iters` back-to-back launches."""
    for i in range(3):
        launch(i % copies)
    ctx.synchronize()
    ctx.timer_start()
    for i in range(iters):
        launch(i % copies)
    return ctx.timer_stop() * 1e3 / iters


def bench_ops(ctx, min_bytes: int = 640 << 20):
    """fp16 decode GEMV (batch 1) and int8/int4 group-quantized matmul (batch 1 and 8) on every projection shape.

    Weights cycle through enough copies (>= 640 MB) that no launch finds its weights in the 256 MB Infinity Cache;
    algorithmic bytes: GEMV 2NK + 2K + 4N, QMM NK bits/8 + 2NK/64 (scales) + 2MK + 4MN."""
    gemv, qmm = [], []
    for name, n, k in OP_SHAPES:
        wbytes = 2 * n * k
        copies = max(2, -(-min_bytes // wbytes))
        iters = 50 if n > 100000 else 200
        w_host = S.synth_normal_f16(7, f"ops.{name}.w", 0.02, n * k)
        dw = ctx.alloc(wbytes * copies)
        for c in range(copies):
            ctx.write(dw + c * wbytes, w_host)
        dx = ctx.upload(S.synth_normal_f16(7, f"ops.{name}.x", 1.0, 8 * k))
        dy = ctx.alloc(8 * n * 4)
        try:
            us = _timed_op(ctx, lambda i: S.gemv_f16(ctx, dw + i * wbytes, dx, dy, n, k), copies, iters)
            alg = 2 * n * k + 2 * k + 4 * n
            gemv.append({"shape": f"{name} {n}x{k}", "us": round(us, 3), "gbs": round(alg / us * 1e-3, 1),
                         "frac": round(alg / us * 1e-3 / HBM_PEAK_GBS, 4)})
        finally:
            ctx.free(dw)
        del w_host
        for bits in (8, 4):
            cbytes = n * k * bits // 8
            sbytes = 2 * n * (k // 64)
            copies = max(2, -(-min_bytes // (cbytes + sbytes)))
            dc = ctx.alloc(cbytes * copies)
            ds = ctx.alloc(sbytes * copies)
            c_host = S.synth_codes(7, f"ops.{name}.codes{bits}", bits, n * k)
            s_host = S.synth_uniform_f16(7, f"ops.{name}.scales{bits}", 0.005, 0.02, n * (k // 64))
            for c in range(copies):
                ctx.write(dc + c * cbytes, c_host)
                ctx.write(ds + c * sbytes, s_host)
            try:
                for m in (1, 8):
                    us = _timed_op(ctx, lambda i: S.qmm(ctx, dx, dc + i * cbytes, bits, ds + i * sbytes, dy, m, n, k),
                                   copies, iters)
                    alg = cbytes + sbytes + 2 * m * k + 4 * m * n
                    qmm.append({"shape": f"{name} {n}x{k}", "bits": bits, "m": m, "us": round(us, 3),
                                "gbs": round(alg / us * 1e-3, 1), "frac": round(alg / us * 1e-3 / HBM_PEAK_GBS, 4)})
            finally:
                ctx.free(dc)
                ctx.free(ds)
        ctx.free(dx)
        ctx.free(dy)
    return gemv, qmm


def _progress(msg: str) -> None:
    """A line on stderr as each stage of the run ends (stdout carries only the result line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _host_threads() -> int:
    """Host threads this process may use (the box gives one GPU's share of its cores)."""
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:  # pragma: no cover
        return max(1, min(16, os.cpu_count() or 1))


def _oracle_layers(O, cfg: S.QwenConfig, layers: int, seed: int):
    """The oracle restatement of a model of cfg's shapes cut to `layers` layers (weights as synth_weights writes
    them for the full model: the seeded generator is counter-based, so a layer's tensors do not depend on the count)."""
    import dataclasses
    small = dataclasses.replace(cfg, num_hidden_layers=layers)
    return O.OracleModel(small, S.synth_weights(small, seed), "port")


def cpu_baseline(cfg: S.QwenConfig):
    """The reference CPU runtime on this host, for each configuration:

    * config 1 (the headline): GenerationSession::Generate of the compiled reference (generation_session.cpp:46-79:
      the 32-token prompt forwarded twice, uncached for the logits and cached for the KV, then 15 cached decode
      steps, the calls GenerationSession::Generate makes, in its order) on one core, as the reference runs (no
      threading anywhere in it); value = 16 tokens / wall time;
    * config 2: Linear::Forward (linear.cpp:51-84) per Qwen3-0.6B projection shape at batch 1, compiled reference;
    * config 3: the group-quantized matmul per shape at batch 1 and 8, int8 and int4: the reference has no such
      kernel, so its restatement (orc_qmm_group), all host threads;
    * config 4: prefill of 2048 tokens, extrapolated: one and two layers of Qwen3-0.6B timed on the restatement
      (bit-identical to the reference, all host threads), the layer time x 28 plus the rest;
    * config 5: one ragged step of the 16 Qwen3-4B sequences, extrapolated: per sequence a single-token cached
      forward of a one-layer Qwen3-4B over its KV length on the restatement (all host threads), the layer part x 36
      plus the LM head, summed over the sequences; x 64 steps for the config's run.
    """
    try:
        from oracle import oracle as O
    except Exception as e:  # pragma: no cover
        return {"value": None, "error": str(e)}
    threads = _host_threads()
    out = {"unit": "tok/s", "cpu_model": _cpu_model(), "nproc": os.cpu_count(), "threads_available": threads}
    # ---- config 1 ----
    kind = "reference" if O.ref_available() else "port"
    O.set_threads(1)
    w = S.synth_weights(cfg, 1)
    om = O.OracleModel(cfg, w, kind)
    del w
    prompt = S.synth_tokens(1, "prompt", cfg.vocab_size, PROMPT)
    # GenerationSession::Generate's calls in its order (generation_session.cpp:46-79): the uncached prompt forward
    # (its last row gives the first token), the cached prompt forward (fills the KV), then one cached single-token
    # forward per further token; greedy sampling is the lowest-index argmax (sampler.cpp:42-48)
    cache = O.RefCache(om, PROMPT + 24) if kind == "reference" else O.OracleCache(om, PROMPT + 24)
    stages = {}
    t0 = time.perf_counter()
    first = om.forward_logits(prompt)[-1]
    stages["prompt_uncached_s"] = time.perf_counter() - t0
    _progress(f"cpu config 1: uncached prompt forward {stages['prompt_uncached_s']:.1f} s")
    t1 = time.perf_counter()
    cache.forward(prompt, 0)
    stages["prompt_cached_s"] = time.perf_counter() - t1
    _progress(f"cpu config 1: cached prompt forward {stages['prompt_cached_s']:.1f} s")
    toks = [int(np.argmax(first))]
    t2 = time.perf_counter()
    for i in range(15):
        row = cache.forward(np.array([toks[-1]], np.int32), PROMPT + i)[-1]
        toks.append(int(np.argmax(row)))
    stages["decode_15_s"] = time.perf_counter() - t2
    gen_s = time.perf_counter() - t0
    _progress(f"cpu config 1: 15 decode steps {stages['decode_15_s']:.1f} s")
    del cache
    om.close()
    out.update({"value": round(16 / gen_s, 4), "cores": 1, "kind": kind,
                "sample": f"config 1 in full: Qwen3-0.6B seed-1 weights, 32-token prompt, 16 greedy tokens as "
                          f"GenerationSession::Generate runs them (prompt forwarded twice, uncached and cached, then "
                          f"15 cached decode steps), one core: {gen_s:.1f} s",
                "generate_s": round(gen_s, 2), **{k: round(v, 2) for k, v in stages.items()},
                "decode_tok_s": round(15 / stages["decode_15_s"], 4), "generated_tokens_head": toks[:4]})
    # ---- config 2 ----
    lin = []
    for name, n, k in OP_SHAPES:
        x = np.random.default_rng(1).standard_normal((1, k)).astype(np.float32)
        wt = S.synth_normal_f16(7, f"ops.{name}.w", 0.02, n * k).reshape(n, k)
        y = np.empty((1, n), np.float32)
        t0 = time.perf_counter()
        if kind == "reference":
            O.ref_lib().ref_linear_f16(x.ctypes.data, 1, k, wt.ctypes.data, n, y.ctypes.data)
        else:
            O.linear_f16(x, wt)
        sec = time.perf_counter() - t0
        lin.append({"shape": f"{name} {n}x{k}", "ms": round(sec * 1e3, 2), "gbs": round(2 * n * k / sec / 1e9, 2)})
    out["config2_linear_bs1"] = {"kind": kind, "cores": 1, "rows": lin}
    # ---- config 3 ----
    qrows = []
    O.set_threads(threads)
    for name, n, k in OP_SHAPES:
        a = S.synth_normal_f16(7, f"ops.{name}.x", 1.0, 8 * k).reshape(8, k)
        for bits in (8, 4):
            codes = S.synth_codes(7, f"ops.{name}.codes{bits}", bits, n * k)
            scales = S.synth_uniform_f16(7, f"ops.{name}.scales{bits}", 0.005, 0.02, n * (k // 64))
            for m in (1, 8):
                t0 = time.perf_counter()
                O.qmm_group(a[:m], codes, bits, scales, k, n)
                sec = time.perf_counter() - t0
                qrows.append({"shape": f"{name} {n}x{k}", "bits": bits, "m": m, "ms": round(sec * 1e3, 2)})
    out["config3_qmm_g64"] = {"kind": "port (no reference kernel)", "cores": threads, "rows": qrows}
    _progress("cpu configs 2 and 3 done")
    # ---- config 4 ----
    O.set_threads(threads)
    ids = S.synth_tokens(4, "prefill", cfg.vocab_size, 2048)
    times = {}
    for layers in (1, 2):
        m = _oracle_layers(O, cfg, layers, 1)
        cache = O.OracleCache(m, 2048)
        t0 = time.perf_counter()
        cache.forward(ids, 0)
        times[layers] = time.perf_counter() - t0
        del cache
        m.close()
    layer_s = times[2] - times[1]
    total4 = times[1] + (cfg.num_hidden_layers - 1) * layer_s
    out["config4_prefill_2048"] = {"kind": "port", "cores": threads, "extrapolated": True,
                                   "one_layer_s": round(layer_s, 3), "prefill_s": round(total4, 2),
                                   "tok_s": round(2048 / total4, 1),
                                   "sample": "Qwen3-0.6B with 1 and 2 layers timed (2048-token cached forward, "
                                             "last-row head); layer = difference, x 28 layers"}
    _progress(f"cpu config 4: one layer at 2048 tokens {layer_s:.1f} s")
    # ---- config 5 ----
    cfg4 = S.QWEN3_4B
    lens = S.synth_int_uniform(5, "ragged.kv_len", RAGGED_MIN, RAGGED_MAX, RAGGED_SEQS)
    toks5 = S.synth_tokens(6, "ragged.tokens", cfg4.vocab_size, RAGGED_SEQS)
    m = _oracle_layers(O, cfg4, 1, 1)
    rng = np.random.default_rng(7)
    kvrow = rng.standard_normal((2, cfg4.num_key_value_heads, cfg4.head_dim)).astype(np.float32)
    step_s = 0.0
    # the LM head alone (one row through the 151936 x 2560 tied embedding), to split the one-layer forward
    xh = np.random.default_rng(2).standard_normal((1, cfg4.hidden_size)).astype(np.float32)
    emb = S.synth_normal_f16(1, "model.embed_tokens.weight", 0.02, cfg4.vocab_size * cfg4.hidden_size)
    t0 = time.perf_counter()
    O.linear_f16(xh, emb.reshape(cfg4.vocab_size, cfg4.hidden_size))
    head_s = time.perf_counter() - t0
    del emb
    for i, n in enumerate(lens):
        cache = O.OracleCache(m, int(n) + 2)
        for pos in range(int(n)):  # the cache's contents do not change the cost; one row repeated
            cache.write(0, pos, kvrow[0], kvrow[1])
        t0 = time.perf_counter()
        cache.forward(np.array([toks5[i]], np.int32), int(n))
        t1 = time.perf_counter() - t0
        del cache
        step_s += cfg4.num_hidden_layers * max(t1 - head_s, 0.0) + head_s
    m.close()
    out["config5_ragged_4b"] = {"kind": "port", "cores": threads, "extrapolated": True,
                                "step_s": round(step_s, 2), "run_64_steps_s": round(64 * step_s, 1),
                                "tok_s": round(RAGGED_SEQS / step_s, 3), "lm_head_s": round(head_s, 3),
                                "sample": "per sequence a single-token cached forward of a 1-layer Qwen3-4B over its "
                                          "KV length (lengths of the GPU run), minus the LM head, x 36 layers, plus "
                                          "the head; summed over the 16 sequences"}
    _progress("cpu config 5 done")
    O.set_threads(1)
    return out


def bench_cpp_api() -> dict | None:
    """The kept C++ host API on the headline workload: soc_amd/apps/soc_generate (GenerationContext::Generate over
    CommandScheduler -> QwenCausalLM::ForwardLogitsCached -> Sampler, Mac/gpu/src/runtime/generation_context.cpp:
    118-172) with the seed-1 Qwen3-0.6B weights and the same 32-token prompt, 16 new tokens, run as a child process
    after this one has released the GPU. Reports its wall-clock Generate time and DecodeNextToken latency."""
    import subprocess
    exe = ROOT / "soc_amd" / "apps" / "soc_generate"
    if not exe.exists():
        return {"error": f"{exe} is not built"}
    args = [str(exe), "--model", "qwen3-0.6b", "--seed", "1", "--sigma", "0.02", "--prompt-seed", "1",
            "--prompt-len", str(PROMPT), "--new", "16", "--repeat", "5", "--decode-steps", "64"]
    r = subprocess.run(args, capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        return {"error": (r.stderr or r.stdout)[-400:]}
    out = json.loads(r.stdout.strip().splitlines()[-1])
    out["workload"] = ("GenerationContext::Generate, Qwen3-0.6B seed-1 weights, 32-token prompt, 16 greedy tokens "
                       "(wall clock, host synchronisation included)")
    out.pop("generate_ms", None)
    return out


TRAFFIC_SUMMARY = {"xcd": ROOT / "profiles" / "k_decode_xcd_qwen3_0p6b_traffic.md",
                   "persistent": ROOT / "profiles" / "k_decode_persistent_qwen3_0p6b_traffic.md"}


def measured_traffic(path: Path, key: str = "traffic_bytes_per_launch"):
    """HBM bytes of a one-launch decode kernel from its committed rocprofv3 counter summary (line `<key>: <int>`;
    the XCD kernel's summary gives them per decode token), or None when no summary exists."""
    try:
        for line in path.read_text().splitlines():
            if line.strip().startswith(key + ":"):
                return int(line.split(":", 1)[1].strip())
    except OSError:
        return None
    return None


# Decode tokens per launch of k_decode_xcd (kXcdStepsPerLaunch in soc_amd/csrc/runtime.cpp): soc_decode_steps runs
# up to this many steps in one launch.
XCD_TOKENS_PER_LAUNCH = 128


def copy_calibrate(mib: int = 1024) -> None:
    """A plain device copy of known size (`mib` MiB read + `mib` MiB written, one elementwise kernel), run under
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE to scale those counters to bytes."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibrate_bytes_read": n * 4, "copy_calibrate_bytes_written": n * 4, "launches": 3}),
          flush=True)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-ragged", action="store_true", help="skip the Qwen3-4B ragged decode measurement")
    ap.add_argument("--no-ops", action="store_true", help="skip the GEMV / group-quantized matmul microbenchmarks")
    ap.add_argument("--no-4b", action="store_true", help="skip the Qwen3-4B batch-1 decode measurement")
    ap.add_argument("--no-quant", action="store_true", help="skip the group-quantized prefill measurement")
    ap.add_argument("--no-cpp-api", action="store_true", help="skip the GenerationContext (C++ API) measurement")
    ap.add_argument("--ragged-steps", type=int, default=RAGGED_STEPS, help="steps of the ragged run (profiling)")
    ap.add_argument("--steps-4b", type=int, default=64, help="timed steps of the Qwen3-4B batch-1 decode")
    ap.add_argument("--prefill-only", action="store_true",
                    help="profiling: only the 2048-token prefill (prints {\"prefill_ms_2048\": ...}, no decode line)")
    ap.add_argument("--copy-calibrate", action="store_true",
                    help="only run a plain copy of known size (for scaling rocprofv3 byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        sys.exit("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)")
    if args.copy_calibrate:
        copy_calibrate()
        return

    cfg = S.QWEN3_0_6B
    ctx = S.Context(0)
    m = S.Model(ctx, cfg).synthesize(1, 0.02)
    if args.prefill_only:
        print(json.dumps({"prefill_ms_2048": round(bench_prefill(ctx, m, cfg, 2048), 3)}), flush=True)
        m.close()
        return
    path = m.decode_path()
    ms, mean_kv, toks = bench_decode(ctx, m, cfg, args.steps, args.warmup)
    _progress(f"decode: {ms / args.steps:.4f} ms per token ({path})")
    ms_per_step = ms / args.steps
    tok_s = 1000.0 / ms_per_step
    bpt = decode_bytes_per_token(cfg, mean_kv)
    step_gbs = bpt / (ms_per_step * 1e-3) / 1e9

    prefill_ms = None if args.no_prefill else bench_prefill(ctx, m, cfg, 2048)
    if prefill_ms is not None:
        _progress(f"prefill of 2048 tokens: {prefill_ms:.3f} ms")
    us, alg = bench_gemv_kernel(ctx)
    gemv_gbs = alg / (us * 1e-6) / 1e9
    m.close()
    prefill_q = None if (args.no_prefill or args.no_quant) else bench_prefill_quant(ctx, cfg)
    if prefill_q is not None:
        _progress(f"quantized prefill of 2048 tokens: int8 {prefill_q['int8_ms']} ms, int4 {prefill_q['int4_ms']} ms")
    ops_gemv, ops_qmm = (None, None) if args.no_ops else bench_ops(ctx)
    ragged = None if args.no_ragged else bench_ragged(ctx, args.ragged_steps)
    if ragged is not None:
        _progress(f"Qwen3-4B ragged step: {ragged['ms_per_step']} ms")
    decode_4b = None if args.no_4b else bench_decode_4b(ctx, args.steps_4b)
    if decode_4b is not None:
        _progress(f"Qwen3-4B decode: {decode_4b['ms_per_token']} ms per token")
    ctx.close()
    cpp_api = None if args.no_cpp_api else bench_cpp_api()
    if cpp_api is not None:
        _progress(f"GenerationContext::Generate: {cpp_api.get('generate_ms_median')} ms for 16 tokens")

    if path == "xcd":
        # the timed steps run as ceil(K / XCD_TOKENS_PER_LAUNCH) launches: the events around them give the average
        # launch duration (the short gaps between launches included) and tpl tokens per launch on average
        tpl = args.steps / -(-args.steps // XCD_TOKENS_PER_LAUNCH)
        per_tok = measured_traffic(TRAFFIC_SUMMARY[path], "traffic_bytes_per_token")
        roofline = {"kernel": f"k_decode_xcd ({tpl:g} decode tokens per launch, each 28 layers + LM head + greedy "
                              "token)",
                    "bound": "hbm", "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(step_gbs / HBM_PEAK_GBS, 4),
                    "traffic": round(per_tok * tpl) if per_tok is not None else None, "tokens_per_launch": tpl,
                    "avg_launch_us": round(ms_per_step * 1e3 * tpl, 3), "alg_bytes_per_launch": round(bpt * tpl)}
    elif path == "persistent":
        # one launch per token
        roofline = {"kernel": "k_decode_persistent (whole decode token: 28 layers + LM head + argmax)",
                    "bound": "hbm", "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(step_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(TRAFFIC_SUMMARY[path]),
                    "avg_launch_us": round(ms_per_step * 1e3, 3), "alg_bytes_per_launch": int(bpt)}
    else:
        roofline = {"kernel": "k_gemv<4,2,EPI_STORE> (decode QKV projection 4096x1024 fp16)", "bound": "hbm",
                    "achieved": round(gemv_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(gemv_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                    "avg_launch_us": round(us, 3), "alg_bytes_per_launch": alg}

    cpu = None if args.no_cpu else cpu_baseline(cfg)
    out = {
        "metric": "decode tok/s + % HBM roofline (Qwen3-0.6B fp16 bs1); prefill tok/s @2048",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 weights, fp32 accumulate",
        "data": "synthetic: random-init fp16 weights N(0,0.02) seed 1, uniform random prompt token ids",
        "config": {"workload": "Qwen3-0.6B (28 layers, hidden 1024, 16 q / 8 kv heads, head_dim 128, "
                               "intermediate 3072, vocab 151936, tied) greedy decode at batch 1 after a 32-token "
                               "prompt", "global_batch": 1, "seq_len": int(mean_kv), "parallelism": "none (1 GPU)"},
        "decode_path": path,
        "decode_bytes_per_token": int(bpt),
        "decode_hbm_gbs": round(step_gbs, 1),
        "decode_hbm_roofline_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "prefill_tok_s": None if prefill_ms is None else round(2048 / (prefill_ms * 1e-3), 1),
        "prefill_ms_2048": None if prefill_ms is None else round(prefill_ms, 3),
        "prefill_quant_2048": prefill_q,
        "prefill_roofline": None if prefill_ms is None else {
            "workload": "2048-token prefill, Qwen3-0.6B: 28 layers (projections, causal attention, norms) and the "
                        "last row's LM head", "bound": "mfma",
            "achieved": round(prefill_flop(cfg, 2048) / (prefill_ms * 1e-3) / 1e12, 1), "peak": FP16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(prefill_flop(cfg, 2048) / (prefill_ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
            "alg_flop": prefill_flop(cfg, 2048)},
        "roofline": roofline,
        "gemv_qkv_4096x1024": {"avg_launch_us": round(us, 3), "gbs": round(gemv_gbs, 1),
                               "frac": round(gemv_gbs / HBM_PEAK_GBS, 4)},
        "gemv_f16_bs1": ops_gemv,
        "qmm_g64": ops_qmm,
        "ragged_4b": ragged,
        "decode_4b": decode_4b,
        "cpp_api_generate": cpp_api,
        "cpu_baseline": cpu,
        "generated_tokens_head": [int(t) for t in toks[:8]],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
