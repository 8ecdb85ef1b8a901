"""Models loaded from bundles on disk (soc_model_load_bundle; QwenModelLoader::LoadModelFromFile through the C++
harness program) on the GPU:
  (1) a float16 bundle of a fixture model generates the reference fixture's tokens and logits;
  (2) a float32 bundle of the same (fp16-exact) values gives the same logits bit for bit;
  (3) a bfloat16 bundle at Qwen3-0.6B layer shapes (3 layers, 8 KV heads, the XCD decode path): prefill and decode
      logits against the oracle run on the weights the loader produced (read back on the CPU through
      soc_bundle_tensor_f16), within the model tolerance;
  (4) the C++ loader + harness call sequence on the float16 bundle equals (1).
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

import soc_amd as S
from tests.bundle import config_dict, write_bundle
from tests.golden.make_golden import SMALL_MODELS
from tests.parity import assert_logits_close

pytestmark = pytest.mark.gpu


def _bundle_of(tmp, cfg, weights, dtype):
    tensors = {name: (w.view(np.uint16) if dtype == "float16" else w.view(np.float16).astype(np.float32), dtype)
               for name, w in weights.items()}
    return write_bundle(tmp, config_dict(cfg, dtype), tensors, export_dtype=dtype)


def _generate(m, prompt, new, plen):
    kv = S.KVCache(m, 1, 64)
    try:
        logits, tok = S.prefill(m, kv, 0, prompt, 0, logit_rows=plen)
        rows, toks = [logits], [tok]
        for _ in range(1, new):
            lg, tok = S.decode(m, kv, 0, toks[-1])
            rows.append(lg[None])
            toks.append(tok)
        return np.concatenate(rows), toks
    finally:
        kv.close()


def test_bundle_generation_matches_reference(gpu_ctx, golden, tmp_path):
    name = "tiny_untied"
    cfg, seed, plen, new = SMALL_MODELS[name]
    g = golden(f"model_{name}.npz")
    w = S.synth_weights(cfg, seed)
    runs = {}
    for dtype in ("float16", "float32"):
        m = S.load_bundle(gpu_ctx, _bundle_of(tmp_path / dtype, cfg, w, dtype))
        try:
            runs[dtype] = _generate(m, g["prompt"], new, plen)
        finally:
            m.close()
    rows, toks = runs["float16"]
    assert toks == g["tokens"].tolist()
    assert_logits_close(rows[:plen], g["prompt_logits"], "bundle prompt rows")
    for i in range(1, new):
        assert_logits_close(rows[plen + i - 1], g["step_logits"][i], f"bundle step {i}")
    assert np.array_equal(runs["float32"][0].view(np.uint32), rows.view(np.uint32))
    assert runs["float32"][1] == toks


def test_bundle_bf16_xcd_shapes_against_oracle(gpu_ctx, oracle_mod, tmp_path):
    cfg = S.QwenConfig(vocab_size=4096, hidden_size=1024, num_hidden_layers=3, num_attention_heads=16,
                       num_key_value_heads=8, intermediate_size=3072, tie_word_embeddings=True)
    w = S.synth_weights(cfg, 21, 0.05)
    path = _bundle_of(tmp_path, cfg, w, "bfloat16")
    b = S.Bundle(path)
    loaded = {name: b.tensor_f16(name, shape) for name, shape in S.tensor_specs(b.config())}
    b.close()
    assert not all(np.array_equal(loaded[n], w[n]) for n in loaded)  # bf16 really rounded something
    m = S.load_bundle(gpu_ctx, path)
    kv = S.KVCache(m, 1, 64)
    try:
        ids = S.synth_tokens(22, "bundle", cfg.vocab_size, 20)
        lg, tok = S.prefill(m, kv, 0, ids)
        om = oracle_mod.OracleModel(cfg, loaded)
        cache = oracle_mod.OracleCache(om, 64)
        ref = cache.forward(ids, 0, logit_rows=1)
        assert_logits_close(lg[0], ref[0], "bf16 bundle prefill")
        assert tok == oracle_mod.sample(ref[0])
        for i in range(3):
            lg, nt = S.decode(m, kv, 0, tok)
            r = cache.forward(np.array([tok], np.int32), 20 + i)
            assert_logits_close(lg, r[0], f"bf16 bundle decode {i}")
            assert nt == oracle_mod.sample(r[0])
            tok = nt
    finally:
        kv.close()
        m.close()


def test_cpp_loader_from_bundle(golden, tmp_path):
    exe = Path(__file__).resolve().parent / "cpp" / "test_harness_sequence"
    name = "tiny_untied"
    cfg, seed, plen, new = SMALL_MODELS[name]
    g = golden(f"model_{name}.npz")
    path = _bundle_of(tmp_path / "b", cfg, S.synth_weights(cfg, seed), "float16")
    out = tmp_path / "h.bin"
    r = subprocess.run([str(exe), str(out), "--bundle", str(path), "1", str(new)] + [str(int(t)) for t in g["prompt"]],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    from tests.test_gpu_host_api import _read_harness
    toks, _, _, rows = _read_harness(out)
    assert toks == g["tokens"].tolist()
    assert_logits_close(rows[:plen], g["prompt_logits"], "C++ bundle loader prompt rows")
