"""Qwen3-1.7B and Qwen3-8B layer widths: per-op decode, one-row ragged decode and prefill.

Above Qwen3-0.6B a batch-1 decode token runs the per-op kernels (the one-launch kernel is limited to hidden 1024 /
intermediate 3072), whose GEMV split, attention chunk and skinny split choices depend on the widths: K = 2048 / 6144
(1.7B) and 4096 / 12288 (8B).
  (1) Two-layer models at those widths (32 q / 8 kv or 16 q / 8 kv heads) with a 4096-token vocabulary against the
      oracle's forward: prompt logits, then greedy steps through soc_decode (per-op graph) and through one-row
      ragged batches (skinny kernels); logits within the model tolerance, identical greedy tokens.
  (2) The full-size models (seeded N(0, 0.02) weights synthesized on the device): per-op decode equals one-row ragged
      decode of the same prompt within the model tolerance, with the same tokens (no oracle: a CPU forward of the
      full 8B model is too slow for the suite).
"""
import numpy as np
import pytest

import soc_amd as S
from tests.parity import assert_logits_close

pytestmark = pytest.mark.gpu

WIDTHS = {"1.7B": S.QWEN3_1_7B, "8B": S.QWEN3_8B}


def _two_layer(full: S.QwenConfig) -> S.QwenConfig:
    return S.QwenConfig(vocab_size=4096, hidden_size=full.hidden_size, num_hidden_layers=2,
                        num_attention_heads=full.num_attention_heads, num_key_value_heads=full.num_key_value_heads,
                        intermediate_size=full.intermediate_size, tie_word_embeddings=full.tie_word_embeddings)


def _decode_both(m, cfg, prompt, steps):
    """(per-op logits rows, tokens), (one-row ragged logits rows, tokens) after prefilling `prompt` in two slots."""
    kv = S.KVCache(m, 2, len(prompt) + steps + 8)
    try:
        out = []
        for slot in (0, 1):
            lg, tok = S.prefill(m, kv, slot, prompt)
            rows, toks = [lg[0]], [tok]
            for _ in range(steps):
                if slot == 0:
                    lg, tok = S.decode(m, kv, 0, toks[-1])
                else:
                    lgb, nxt = S.decode_batch(m, kv, np.array([1], np.int32), np.array([toks[-1]], np.int32))
                    lg, tok = lgb[0], int(nxt[0])
                rows.append(lg)
                toks.append(tok)
            out.append((rows, toks))
        return out
    finally:
        kv.close()


@pytest.mark.parametrize("name", list(WIDTHS))
def test_two_layer_widths_match_oracle(gpu_ctx, oracle_mod, name):
    cfg = _two_layer(WIDTHS[name])
    w = S.synth_weights(cfg, 41)
    m = S.Model(gpu_ctx, cfg).load(w)
    prompt = S.synth_tokens(42, "sizes.prompt", cfg.vocab_size, 12)
    try:
        assert m.decode_path() == "graph"
        (ra, ta), (rb, tb) = _decode_both(m, cfg, prompt, 3)
    finally:
        m.close()
    om = oracle_mod.OracleModel(cfg, w)
    try:
        want, want_lg = om.generate(prompt, 4, want_logits=True)
    finally:
        om.close()
    assert ta == want.tolist() and tb == want.tolist()
    for i in range(4):
        assert_logits_close(ra[i], want_lg[i], f"{name} widths, 2 layers, per-op step {i}")
        assert_logits_close(rb[i], want_lg[i], f"{name} widths, 2 layers, ragged step {i}")


@pytest.mark.parametrize("name", list(WIDTHS))
def test_full_size_per_op_decode_equals_ragged(gpu_ctx, name):
    cfg = WIDTHS[name]
    m = S.Model(gpu_ctx, cfg).synthesize(43, 0.02)
    prompt = S.synth_tokens(44, "sizes.full", cfg.vocab_size, 16)
    try:
        assert m.decode_path() == "graph"
        (ra, ta), (rb, tb) = _decode_both(m, cfg, prompt, 4)
    finally:
        m.close()
    assert ta == tb
    for i in range(5):
        assert_logits_close(ra[i], rb[i], f"Qwen3-{name} per-op vs ragged step {i}")
