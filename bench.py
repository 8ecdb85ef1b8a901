#!/usr/bin/env python3
"""Benchmark of the Qwen3 forward hot path on one MI355X.

Workload (headline): Qwen3-0.6B architecture, random-init fp16 weights N(0, 0.02) (seed 1), batch 1. A 32-token
prompt is prefilled (untimed), then W warmup and K timed greedy decode steps run with the sampled token fed back on
the device. A "step" is one decode token. Also measured in the same run:
  * prefill of a 2048-token prompt (tok/s),
  * the dominant decode kernel: k_decode_xcd (one launch = one whole token, every layer split over the 8 XCDs) or
    k_decode_persistent when the device runs that one, timed with HIP events on the stream it is launched on; the
    fused RMSNorm + QKV GEMV
    (4096 x 1024 fp16, over weight copies larger than the 256 MB Infinity Cache) is reported beside it,
  * every decode projection shape (q, k/v, o, gate/up, down, LM head) as an fp16 GEMV at batch 1 and as the
    int8 / int4 group-quantized matmul (group 64, fp16 scales) at batch 1 and 8, in GB/s against 8 TB/s,
  * the Qwen3-4B ragged decode batch (16 sequences, seeded KV lengths in [64, 4096]),
  * Qwen3-4B greedy decode at batch 1 (per-op kernels replayed as a HIP graph),
  * the reference CPU runtime (compiled reference sources when available, else the oracle restatement), on the
    host, one core, on a bounded sample.
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


def bench_ragged(ctx):
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
        warm = S.decode_batch_steps(m, kv, slots, toks, RAGGED_STEPS)  # builds and replays the step graph
        start = [kv.length(int(i)) for i in slots]
        ctx.synchronize()
        ctx.timer_start()
        out = S.decode_batch_steps(m, kv, slots, warm[-1], RAGGED_STEPS)
        ms = ctx.timer_stop()
    finally:
        kv.close()
        m.close()
    per_step = ms / RAGGED_STEPS
    mean_bytes = np.mean([ragged_bytes_per_step(cfg, [s + t for s in start]) for t in range(RAGGED_STEPS)])
    gbs = mean_bytes / (per_step * 1e-3) / 1e9
    return {"workload": "Qwen3-4B ragged decode, 16 sequences, KV lengths U[64,4096] (seed 5), 64 steps",
            "kv_lengths": [int(x) for x in lens], "tok_s": round(RAGGED_SEQS * RAGGED_STEPS / (ms * 1e-3), 1),
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


def cpu_baseline(cfg: S.QwenConfig, budget_s: float = 20.0):
    """The reference CPU runtime on a bounded sample: single-token cached forwards of the full model."""
    try:
        from oracle import oracle as O
    except Exception as e:  # pragma: no cover
        return {"value": None, "error": str(e)}
    kind = "reference" if O.ref_available() else "port"
    O.set_threads(1)
    w = S.synth_weights(cfg, 1)
    om = O.OracleModel(cfg, w, kind)
    ids = S.synth_tokens(1, "prompt", cfg.vocab_size, 1)
    times = []
    t_start = time.time()
    while len(times) < 5 and (time.time() - t_start) < budget_s:
        if kind == "reference":
            lib = O.ref_lib()
            c = lib.ref_cache_create(om.h, 4)
            logits = np.empty((1, cfg.vocab_size), np.float32)
            t0 = time.perf_counter()
            rc = lib.ref_forward_logits_cached(om.h, c, ids.ctypes.data, 1, 0, logits.ctypes.data)
            times.append(time.perf_counter() - t0)
            lib.ref_cache_destroy(c)
            if rc != 0:
                return {"value": None, "error": lib.ref_last_error().decode()}
        else:
            cache = O.OracleCache(om, 4)
            t0 = time.perf_counter()
            cache.forward(ids, 0)
            times.append(time.perf_counter() - t0)
    om.close()
    sec = float(np.median(times))
    return {"value": round(1.0 / sec, 4), "unit": "tok/s", "cores": 1, "kind": kind,
            "sample": f"{len(times)} single-token cached forwards of the full {cfg.num_hidden_layers}-layer model "
                      f"(one decode step each; median {sec:.3f} s), 1 host thread of {os.cpu_count()}"}


TRAFFIC_SUMMARY = {"xcd": ROOT / "profiles" / "k_decode_xcd_qwen3_0p6b_traffic.md",
                   "persistent": ROOT / "profiles" / "k_decode_persistent_qwen3_0p6b_traffic.md"}


def measured_traffic(path: Path):
    """HBM bytes per launch of a one-launch decode kernel from its committed rocprofv3 counter summary
    (line `traffic_bytes_per_launch: <int>`), or None when no summary exists."""
    try:
        for line in path.read_text().splitlines():
            if line.strip().startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except OSError:
        return None
    return None


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
    path = m.decode_path()
    ms, mean_kv, toks = bench_decode(ctx, m, cfg, args.steps, args.warmup)
    ms_per_step = ms / args.steps
    tok_s = 1000.0 / ms_per_step
    bpt = decode_bytes_per_token(cfg, mean_kv)
    step_gbs = bpt / (ms_per_step * 1e-3) / 1e9

    prefill_ms = None if args.no_prefill else bench_prefill(ctx, m, cfg, 2048)
    us, alg = bench_gemv_kernel(ctx)
    gemv_gbs = alg / (us * 1e-6) / 1e9
    m.close()
    ops_gemv, ops_qmm = (None, None) if args.no_ops else bench_ops(ctx)
    ragged = None if args.no_ragged else bench_ragged(ctx)
    decode_4b = None if args.no_4b else bench_decode_4b(ctx)
    ctx.close()

    if path in ("xcd", "persistent"):
        # one launch per token: the events around the K launches give the average launch duration (the short
        # gaps between back-to-back launches included)
        kname = "k_decode_xcd" if path == "xcd" else "k_decode_persistent"
        roofline = {"kernel": f"{kname} (whole decode token: 28 layers + LM head + argmax)",
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
        "roofline": roofline,
        "gemv_qkv_4096x1024": {"avg_launch_us": round(us, 3), "gbs": round(gemv_gbs, 1),
                               "frac": round(gemv_gbs / HBM_PEAK_GBS, 4)},
        "gemv_f16_bs1": ops_gemv,
        "qmm_g64": ops_qmm,
        "ragged_4b": ragged,
        "decode_4b": decode_4b,
        "cpu_baseline": cpu,
        "generated_tokens_head": [int(t) for t in toks[:8]],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
