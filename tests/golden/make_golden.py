"""Writes the golden fixtures under tests/golden/ from the reference's own CPU sources.

Runs only where the reference checkout exists: `make -C oracle ref` compiles /root/reference/Mac/cpu/src (the
13 hot-path files) plus oracle/ref_driver.cpp into oracle/_ref/libsocref.so, and this script drives it. The
fixtures are data (inputs and outputs); the GPU tests and the CPU test suite read them without the reference.

Fixtures:
  dtype_f16.npz     Float16ToFloat32 (Mac/cpu/src/dtype.cpp:76-106) of all 65,536 codes, and Float32ToFloat16
                    (:115-156) of a fixed set of floats including subnormals, overflow and rounding ties.
  ops_small.npz     Linear / RMSNorm / RoPE / GQA / Sampler outputs on small seeded inputs.
  quant_int8.npz    QuantizeMatMulRhs8 + MatMulQuantized (Mac/cpu/header/matrix_ops.h:42-74, :308-350).
  model_<name>.npz  Greedy generation (GenerationSession::Generate semantics) of small random Qwen3 models:
                    prompt, generated tokens and every step's full logits row.
  qwen3_0p6b.npz    Qwen3-0.6B architecture, weights N(0, 0.02) seed 1, 32-token prompt (seed 1), 16 greedy tokens.
                    Per step: the 64 largest logits (ids, values), logits at 512 seeded indices, and row statistics.
  qwen3_0p6b_s2.npz Qwen3-0.6B architecture, tied, weights N(0, 0.05) seed 2, 32-token prompt (seed 2), 16 greedy
                    tokens, all distinct (the seed-1 model repeats one token), same per-step contents.
  prefill2048.npz   Qwen3-0.6B (seed 1 weights) prefill of the 2048 uniform-random ids synth_tokens(4, "prefill"):
                    the last row's 64 largest logits, logits at 512 seeded indices, argmax and row statistics.
                    Written by this repository's C restatement of the reference (oracle/soc_oracle.cpp) on 8 threads:
                    the compiled reference needs about an hour for one 2048-token forward on one core. Before it
                    writes the fixture the script checks, on a 256-token prefill of the same model (all 28 layers),
                    that the restatement's last-row logits equal the compiled reference's bit for bit.
  ragged4b.npz      Qwen3-4B architecture (tied, seed 1 weights N(0, 0.02)): one decode step of four of the 16
                    sequences of the ragged batch (KV lengths synth_int_uniform(5, "ragged.kv_len", 64, 4096),
                    cache contents N(0, 1) fp16 as soc_kv_fill_synthetic(slot, length, 7) writes them, tokens
                    synth_tokens(6, "ragged.tokens")): the longest, the shortest, and slots 0 and 1. Per sequence
                    the slot, length, token, 64 largest logits, logits at 512 seeded indices and argmax, from the
                    compiled reference.

Usage: python tests/golden/make_golden.py [--skip-0p6b] [--only NAME[,NAME...]]
       (names: dtype, ops, quant, small, 0p6b, 0p6b_s2, prefill2048, ragged4b)
"""
from __future__ import annotations

import argparse
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402
from soc_amd import (QWEN3_0_6B, QWEN3_4B, QwenConfig, synth_int_uniform, synth_normal_f16,  # noqa: E402
                     synth_tokens, synth_weights)

OUT = Path(__file__).resolve().parent

SMALL_MODELS = {
    # name: (config, weight seed, prompt length, new tokens)
    "tiny_tied": (QwenConfig(vocab_size=512, hidden_size=256, num_hidden_layers=2, num_attention_heads=4,
                             num_key_value_heads=2, intermediate_size=512), 11, 12, 8),
    "tiny_untied": (QwenConfig(vocab_size=768, hidden_size=256, num_hidden_layers=3, num_attention_heads=4,
                               num_key_value_heads=2, intermediate_size=384, tie_word_embeddings=False), 12, 9, 10),
    "tiny_g4": (QwenConfig(vocab_size=640, hidden_size=512, num_hidden_layers=2, num_attention_heads=8,
                           num_key_value_heads=2, intermediate_size=1024, tie_word_embeddings=False), 13, 20, 6),
    # eight KV heads like every Qwen3 model: decode takes the XCD-partitioned kernel on MI355X
    "tiny_kv8": (QwenConfig(vocab_size=512, hidden_size=256, num_hidden_layers=2, num_attention_heads=16,
                            num_key_value_heads=8, intermediate_size=768, tie_word_embeddings=False), 14, 11, 9),
    # eight query heads on one KV head: the largest grouping the kernels accept (untied: varied greedy tokens)
    "tiny_g8": (QwenConfig(vocab_size=384, hidden_size=256, num_hidden_layers=2, num_attention_heads=8,
                           num_key_value_heads=1, intermediate_size=512, tie_word_embeddings=False), 15, 13, 7),
}


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return bits.astype(np.uint16).view(np.float16).astype(np.float32)


def write_dtype(ref) -> None:
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f32 = np.empty(65536, dtype=np.float32)
    ref.ref_f16_to_f32_array(codes.ctypes.data, f32.ctypes.data, codes.size)
    rng = np.random.default_rng(5)
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6, 6.1035156e-05, 5.9604645e-08,
                        2.980232e-08, 2.9802326e-08, 1e-9, 0.1, 0.2, 0.3, 1.0009765625, 1.00048828125,
                        1.000732421875, 3.14159265, np.inf, -np.inf, np.nan], dtype=np.float32)
    floats = np.concatenate([special, rng.normal(0, 1, 2000).astype(np.float32),
                             rng.normal(0, 1e-5, 500).astype(np.float32),
                             (rng.normal(0, 1, 500) * 1e4).astype(np.float32)])
    f16 = np.empty(floats.size, dtype=np.uint16)
    ref.ref_f32_to_f16_array(floats.ctypes.data, f16.ctypes.data, floats.size)
    np.savez_compressed(OUT / "dtype_f16.npz", f16_to_f32_bits=f32.view(np.uint32), f32_inputs=floats,
                        f32_to_f16_bits=f16)


def write_ops(ref) -> None:
    rng = np.random.default_rng(7)
    C = O.C
    out = {}
    # Linear: x [3][96] fp32, W fp16 [40][96]
    x = rng.normal(0, 1, (3, 96)).astype(np.float32)
    w = synth_normal_f16(3, "ops.linear.w", 0.05, 40 * 96).reshape(40, 96)
    y = np.empty((3, 40), dtype=np.float32)
    assert ref.ref_linear_f16(x.ctypes.data, 3, 96, w.ctypes.data, 40, y.ctypes.data) == 0
    out.update(linear_x=x, linear_w=w, linear_y=y)
    # RMSNorm: x [5][64], gain fp16 [64]
    x = rng.normal(0, 2, (5, 64)).astype(np.float32)
    g = synth_normal_f16(3, "ops.rms.g", 0.5, 64)
    y = np.empty_like(x)
    assert ref.ref_rmsnorm_f16(x.ctypes.data, 5, 64, g.ctypes.data, np.float32(1e-6), y.ctypes.data) == 0
    out.update(rms_x=x, rms_g=g, rms_y=y)
    # RoPE: [6][3][128] at offset 1000, theta 1e6
    x = rng.normal(0, 1, (6, 3, 128)).astype(np.float32)
    y = x.copy()
    assert ref.ref_rope(y.ctypes.data, 6, 3, 128, 1e6, 1000) == 0
    out.update(rope_x=x, rope_y=y)
    # GQA: T=5 queries after a prefix of 7, nq=4, nkv=2, d=16
    q = rng.normal(0, 1, (5, 4, 16)).astype(np.float32)
    k = rng.normal(0, 1, (12, 2, 16)).astype(np.float32)
    v = rng.normal(0, 1, (12, 2, 16)).astype(np.float32)
    o = np.empty_like(q)
    assert ref.ref_gqa(q.ctypes.data, k.ctypes.data, v.ctypes.data, 5, 12, 4, 2, 16, 7, 1, o.ctypes.data) == 0
    out.update(gqa_q=q, gqa_k=k, gqa_v=v, gqa_o=o)
    # Sampler: top-k with ties
    row = np.array([0.5, 2.0, -1.0, 2.0, 1.5, 2.0, 0.0], dtype=np.float32)
    picks = np.array([ref.ref_sample(row.ctypes.data, row.size, 1.0, kk) for kk in (1, 2, 3, 7)], dtype=np.int32)
    row2 = rng.normal(0, 1, 1000).astype(np.float32)
    picks2 = np.array([ref.ref_sample(row2.ctypes.data, row2.size, t, kk) for t, kk in ((1.0, 1), (0.7, 5), (2.0, 50))],
                      dtype=np.int32)
    out.update(sample_row=row, sample_picks=picks, sample_row2=row2, sample_picks2=picks2)
    np.savez_compressed(OUT / "ops_small.npz", **out)


def write_quant(ref) -> None:
    rng = np.random.default_rng(9)
    a = rng.normal(0, 1, (3, 128)).astype(np.float32)
    rhs = rng.normal(0, 0.05, (128, 24)).astype(np.float32)
    rhs[:, 5] = 0.0  # an all-zero column gets scale 0 and output 0
    codes = np.empty((24, 128), dtype=np.int8)
    scales = np.empty(24, dtype=np.float32)
    y = np.empty((3, 24), dtype=np.float32)
    assert ref.ref_quant_matmul_int8(a.ctypes.data, 3, 128, rhs.ctypes.data, 24, codes.ctypes.data,
                                     scales.ctypes.data, y.ctypes.data) == 0
    np.savez_compressed(OUT / "quant_int8.npz", a=a, rhs=rhs, codes=codes, scales=scales, y=y)


def write_small_models() -> None:
    for name, (cfg, seed, plen, new) in SMALL_MODELS.items():
        w = synth_weights(cfg, seed)
        prompt = synth_tokens(seed, "prompt", cfg.vocab_size, plen)
        m = O.OracleModel(cfg, w, "reference")
        toks, logits = m.generate(prompt, new, want_logits=True)
        full = m.forward_logits(prompt)
        np.savez_compressed(OUT / f"model_{name}.npz", seed=np.int64(seed), prompt=prompt, tokens=toks,
                            step_logits=logits, prompt_logits=full)
        print(name, toks.tolist(), flush=True)


def row_summary(logits: np.ndarray, vocab: int) -> dict[str, np.ndarray]:
    """The parts of full-vocabulary logit rows a fixture keeps: the 64 largest (ids, values), 512 seeded samples,
    and per-row sum, sum of squares and maximum."""
    logits = np.atleast_2d(logits)
    idx = np.sort(np.unique(synth_tokens(1, "fixture.sample", vocab, 600)))[:512].astype(np.int32)
    top_ids = np.argsort(-logits, axis=1, kind="stable")[:, :64].astype(np.int32)
    top_vals = np.take_along_axis(logits, top_ids, axis=1)
    stats = np.stack([logits.astype(np.float64).sum(1), (logits.astype(np.float64) ** 2).sum(1),
                      logits.max(1).astype(np.float64)], axis=1)
    return dict(top_ids=top_ids, top_vals=top_vals, sample_idx=idx, sample_vals=logits[:, idx], stats=stats)


def write_0p6b() -> None:
    cfg = QWEN3_0_6B
    t0 = time.time()
    w = synth_weights(cfg, 1)
    prompt = synth_tokens(1, "prompt", cfg.vocab_size, 32)
    m = O.OracleModel(cfg, w, "reference")
    toks, logits = m.generate(prompt, 16, want_logits=True)
    np.savez_compressed(OUT / "qwen3_0p6b.npz", weight_seed=np.int64(1), prompt=prompt, tokens=toks,
                        **row_summary(logits, cfg.vocab_size))
    print("qwen3-0.6b", toks.tolist(), f"{time.time() - t0:.1f}s", flush=True)


def write_0p6b_s2() -> None:
    cfg, seed, sigma = QWEN3_0_6B, 2, 0.05
    t0 = time.time()
    w = synth_weights(cfg, seed, sigma)
    prompt = synth_tokens(seed, "prompt", cfg.vocab_size, 32)
    m = O.OracleModel(cfg, w, "reference")
    toks, logits = m.generate(prompt, 16, want_logits=True)
    assert len(set(toks.tolist())) == len(toks), "the fixture is meant to have distinct greedy tokens"
    np.savez_compressed(OUT / "qwen3_0p6b_s2.npz", weight_seed=np.int64(seed), sigma=np.float32(sigma), prompt=prompt,
                        tokens=toks, **row_summary(logits, cfg.vocab_size))
    print("qwen3-0.6b seed 2", toks.tolist(), f"{time.time() - t0:.1f}s", flush=True)


def write_prefill2048() -> None:
    cfg = QWEN3_0_6B
    t0 = time.time()
    w = synth_weights(cfg, 1)
    ids = synth_tokens(4, "prefill", cfg.vocab_size, 2048)
    O.set_threads(8)
    port = O.OracleModel(cfg, w, "port")
    # pin the restatement at this model's full depth against the compiled reference (256-token prefill, last row)
    ref = O.OracleModel(cfg, w, "reference")
    want = ref.forward_logits(ids[:256])[-1]
    ref.close()
    cache = O.OracleCache(port, 256)
    got = cache.forward(ids[:256], 0, 1)[0]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "port and reference differ at 256 tokens"
    print(f"prefill2048: restatement == reference at 256 tokens ({time.time() - t0:.1f}s)", flush=True)
    cache = O.OracleCache(port, 2048)
    row = cache.forward(ids, 0, 1)[0]
    np.savez_compressed(OUT / "prefill2048.npz", weight_seed=np.int64(1), ids_seed=np.int64(4), n=np.int64(2048),
                        argmax=np.int32(int(np.argmax(row))), **row_summary(row, cfg.vocab_size))
    print("prefill2048 argmax", int(np.argmax(row)), f"{time.time() - t0:.1f}s", flush=True)


def write_ragged4b() -> None:
    cfg = QWEN3_4B
    t0 = time.time()
    w = synth_weights(cfg, 1)
    lens = synth_int_uniform(5, "ragged.kv_len", 64, 4096, 16)
    toks = synth_tokens(6, "ragged.tokens", cfg.vocab_size, 16)
    slots = sorted({int(np.argmax(lens)), int(np.argmin(lens)), 0, 1})
    ref = O.OracleModel(cfg, w, "reference")
    L, nkv, d = cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim
    rows = []
    for slot in slots:
        n = int(lens[slot])
        cache = O.RefCache(ref, n + 1)
        for layer in range(L):
            k = np.stack([synth_normal_f16(7, f"kv.{slot}.{layer}.{h}.k", 1.0, n * d).reshape(n, d) for h in range(nkv)],
                         axis=1)
            v = np.stack([synth_normal_f16(7, f"kv.{slot}.{layer}.{h}.v", 1.0, n * d).reshape(n, d) for h in range(nkv)],
                         axis=1)
            kf = O.f16_to_f32(k)
            vf = O.f16_to_f32(v)
            for p in range(n):
                cache.write(layer, p, kf[p], vf[p])
        rows.append(cache.forward(toks[slot:slot + 1], n)[0])
        cache.close()
        print(f"ragged4b slot {slot} (kv {n}): argmax {int(np.argmax(rows[-1]))} ({time.time() - t0:.1f}s)", flush=True)
    logits = np.stack(rows)
    np.savez_compressed(OUT / "ragged4b.npz", weight_seed=np.int64(1), slots=np.array(slots, np.int32),
                        kv_lens=lens.astype(np.int32), tokens=toks, argmax=np.argmax(logits, axis=1).astype(np.int32),
                        **row_summary(logits, cfg.vocab_size))


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--skip-0p6b", action="store_true")
    ap.add_argument("--only", default="", help="comma-separated fixture names")
    args = ap.parse_args()
    O.build(ref=True)
    if not O.ref_available():
        sys.exit("the reference library could not be built (is /root/reference present?)")
    ref = O.ref_lib()
    writers = {"dtype": lambda: write_dtype(ref), "ops": lambda: write_ops(ref), "quant": lambda: write_quant(ref),
               "small": write_small_models, "0p6b": write_0p6b, "0p6b_s2": write_0p6b_s2,
               "prefill2048": write_prefill2048, "ragged4b": write_ragged4b}
    heavy = ["0p6b", "0p6b_s2", "prefill2048", "ragged4b"]
    names = [n for n in args.only.split(",") if n] or [n for n in writers if not (args.skip_0p6b and n in heavy)]
    for n in names:
        writers[n]()


if __name__ == "__main__":
    main()
