"""Runs the C++ host-interface programs (tests/cpp) on the GPU.

test_generation_context: the reference's identity-model generation test through GenerationContext.
test_kv_cache: KVCache appends, per-layer lengths, layer views and error messages.
test_harness_sequence: the reference parity harness's call sequence (test_real_bundle_regression.mm) on seeded
models; its prompt logits (all rows, as RunPrefill writes them), step logits and greedy tokens are compared with the
fixtures the compiled reference wrote for the same models, and its top-k lists with the reference sampler on the
rows it produced.
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from tests.golden.make_golden import SMALL_MODELS
from tests.parity import assert_logits_close

pytestmark = pytest.mark.gpu

CPP = Path(__file__).resolve().parent / "cpp"


def test_generation_context_cpp():
    exe = CPP / "test_generation_context"
    assert exe.exists(), "build it with `python -m soc_amd.build` (build_cpp_tests)"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "test_generation_context passed" in r.stdout


def test_kv_cache_cpp():
    exe = CPP / "test_kv_cache"
    assert exe.exists(), "build it with `python -m soc_amd.build` (build_cpp_tests)"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "test_kv_cache passed" in r.stdout


def _read_harness(path):
    raw = np.fromfile(path, dtype=np.int32)
    ng, k = int(raw[0]), int(raw[1])
    o = 2
    toks, ids, vals = [], [], []
    for _ in range(ng):
        toks.append(int(raw[o]))
        ids.append(raw[o + 1:o + 1 + k].copy())
        vals.append(raw[o + 1 + k:o + 1 + 2 * k].view(np.float32).copy())
        o += 1 + 2 * k
    nr, v = int(raw[o]), int(raw[o + 1])
    rows = raw[o + 2:o + 2 + nr * v].view(np.float32).reshape(nr, v)
    return toks, ids, vals, rows


@pytest.mark.parametrize("name", list(SMALL_MODELS))
@pytest.mark.parametrize("top_k", [1, 5])
def test_harness_sequence_matches_reference(golden, oracle_mod, tmp_path, name, top_k):
    exe = CPP / "test_harness_sequence"
    assert exe.exists(), "build it with `python -m soc_amd.build` (build_cpp_tests)"
    cfg, seed, plen, new = SMALL_MODELS[name]
    g = golden(f"model_{name}.npz")
    out = tmp_path / "harness.bin"
    args = [str(exe), str(out), str(cfg.vocab_size), str(cfg.hidden_size), str(cfg.num_hidden_layers),
            str(cfg.num_attention_heads), str(cfg.num_key_value_heads), str(cfg.intermediate_size),
            str(int(cfg.tie_word_embeddings)), str(seed), str(top_k), str(new)] + [str(int(t)) for t in g["prompt"]]
    r = subprocess.run(args, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    toks, ids, vals, rows = _read_harness(out)
    assert_logits_close(rows[:plen], g["prompt_logits"], f"{name} harness prompt rows")
    for i in range(1, new):
        assert_logits_close(rows[plen + i - 1], g["step_logits"][i], f"{name} harness step {i}")
    # each step's sample is over the row the harness read back (the prompt's last row, then each decode row)
    sampled_rows = [rows[plen - 1]] + [rows[plen + i - 1] for i in range(1, new)]
    for s, row in enumerate(sampled_rows):
        rtok, rids, rvals = oracle_mod.sample_topk(row, 1.0, top_k)
        assert toks[s] == rtok and np.array_equal(ids[s], rids), f"step {s}"
        assert np.array_equal(vals[s].view(np.uint32), rvals.view(np.uint32)), f"step {s}"
    if top_k == 1:
        assert toks == g["tokens"].tolist()


def test_qwen_causal_lm_cpp():
    """The reference generation test's call shape with a model built from device weight tensors
    (QwenCausalLM(QwenCausalLMWeights, QwenCausalLMParams), weights()), the four forwards, and the op classes."""
    exe = CPP / "test_qwen_causal_lm"
    assert exe.exists(), "build it with `python -m soc_amd.build` (build_cpp_tests)"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "test_qwen_causal_lm passed" in r.stdout


def test_generation_context_qwen3_0p6b_matches_reference(golden):
    """GenerationContext::Generate (generation_context.cpp:118-172) at Qwen3-0.6B shape: the 16 greedy tokens of the
    compiled reference on the seed-2 N(0, 0.05) model and its 32-token prompt (qwen3_0p6b_s2.npz, 16 distinct
    tokens), through soc_generate, the program that drives the kept C++ API."""
    import json
    g = golden("qwen3_0p6b_s2.npz")
    exe = CPP.parent.parent / "soc_amd" / "apps" / "soc_generate"
    assert exe.exists(), "build it with `python -m soc_amd.build` (build_cpp_tests)"
    args = [str(exe), "--model", "qwen3-0.6b", "--seed", str(int(g["weight_seed"])), "--sigma", str(float(g["sigma"])),
            "--prompt-seed", str(int(g["weight_seed"])), "--prompt-len", "32", "--new", "16", "--repeat", "1",
            "--decode-steps", "4"]
    r = subprocess.run(args, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["tokens"] == g["tokens"].tolist()
