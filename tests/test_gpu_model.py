"""End-to-end parity of the HIP Qwen3 forward (prefill + decode through the fp16 KV cache) on an MI355X.

Checks against (1) golden fixtures written by the reference's own compiled CPU sources (tests/golden), and
(2) the CPU oracle run live on the same seeded inputs. Tolerance (logits, fp32 compute with fp16 weights and an fp16
KV cache): max |gpu - ref| <= 2e-2 and max |gpu - ref| / max |ref| <= 1e-2; greedy tokens must be identical.
"""
import numpy as np
import pytest

import soc_amd as S
from tests.parity import assert_logits_close
from tests.golden.make_golden import SMALL_MODELS

pytestmark = pytest.mark.gpu

def _gpu_model(ctx, cfg, weights):
    return S.Model(ctx, cfg).load(weights)


@pytest.mark.parametrize("name", list(SMALL_MODELS))
def test_small_model_generation_matches_reference(gpu_ctx, golden, name):
    cfg, seed, plen, new = SMALL_MODELS[name]
    g = golden(f"model_{name}.npz")
    m = _gpu_model(gpu_ctx, cfg, S.synth_weights(cfg, seed))
    kv = S.KVCache(m, 1, 64)
    try:
        prompt = g["prompt"]
        logits, tok = S.prefill(m, kv, 0, prompt, 0, logit_rows=plen)
        assert_logits_close(logits, g["prompt_logits"], f"{name} prompt rows")
        toks = [tok]
        assert_logits_close(logits[-1], g["step_logits"][0], f"{name} step 0")
        for i in range(1, new):
            lg, tok = S.decode(m, kv, 0, toks[-1])
            assert_logits_close(lg, g["step_logits"][i], f"{name} step {i}")
            toks.append(tok)
        assert toks == g["tokens"].tolist()
        assert kv.length(0) == plen + new - 1
    finally:
        kv.close()
        m.close()


def test_chunked_prefill_equals_single_prefill(gpu_ctx):
    cfg, seed, _, _ = SMALL_MODELS["tiny_untied"]
    m = _gpu_model(gpu_ctx, cfg, S.synth_weights(cfg, seed))
    ids = S.synth_tokens(5, "chunk", cfg.vocab_size, 40)
    a = S.KVCache(m, 1, 64)
    b = S.KVCache(m, 1, 64)
    try:
        la, ta = S.prefill(m, a, 0, ids, 0, logit_rows=12)
        S.prefill(m, b, 0, ids[:17], 0, logit_rows=0)
        S.prefill(m, b, 0, ids[17:29], 17, logit_rows=0)
        lb, tb = S.prefill(m, b, 0, ids[29:], 29, logit_rows=11)
        # rows are computed independently by the same kernels: bit-identical
        assert np.array_equal(la[1:], lb) and ta == tb
        ka, va = a.read(0, 1)
        kb, vb = b.read(0, 1)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    finally:
        a.close()
        b.close()
        m.close()


def test_decode_matches_prefill_rows(gpu_ctx):
    """Token-by-token decode (GEMV path) reproduces the prefill (GEMM path) logits of the same rows."""
    cfg, seed, _, _ = SMALL_MODELS["tiny_g4"]
    m = _gpu_model(gpu_ctx, cfg, S.synth_weights(cfg, seed))
    ids = S.synth_tokens(6, "dec", cfg.vocab_size, 24)
    a = S.KVCache(m, 1, 32)
    b = S.KVCache(m, 1, 32)
    try:
        full, _ = S.prefill(m, a, 0, ids, 0, logit_rows=24)
        S.prefill(m, b, 0, ids[:10], 0, logit_rows=0)
        for t in range(10, 24):
            lg, _ = S.decode(m, b, 0, int(ids[t]))
            assert_logits_close(lg, full[t], f"row {t}")
    finally:
        a.close()
        b.close()
        m.close()


@pytest.mark.parametrize("nq,nkv", [(2, 2), (4, 2), (8, 2)])
def test_prefill_mfma_attention_matches_row_kernel(gpu_ctx, monkeypatch, nq, nkv):
    """Both MFMA flash prefill attention kernels (q and p carried as fp16 hi/lo pairs; the default one balances
    pairs of query tiles for 2 or 4 q heads per kv head, SOC_PREFILL_ATTN=tiles selects the per-tile one) agree with
    the per-row fp32 kernel to well inside fp32 noise x depth: max |diff| <= 1e-3 * max |logit| over every row, for
    a single prefill and for a chunked one whose chunk starts off the 32-key tile grid (positions 70.., rows 0..79
    of the chunk)."""
    cfg = S.QwenConfig(vocab_size=384, hidden_size=256, num_hidden_layers=2, num_attention_heads=nq,
                       num_key_value_heads=nkv, intermediate_size=512, tie_word_embeddings=False)
    m = _gpu_model(gpu_ctx, cfg, S.synth_weights(cfg, 11))
    ids = S.synth_tokens(12, "fa", cfg.vocab_size, 150)
    runs = {}
    try:
        for mode in ("rows", "tiles", "mfma"):
            if mode == "mfma":
                monkeypatch.delenv("SOC_PREFILL_ATTN", raising=False)
            else:
                monkeypatch.setenv("SOC_PREFILL_ATTN", mode)
            kv = S.KVCache(m, 1, 160)
            try:
                full, tok = S.prefill(m, kv, 0, ids, 0, logit_rows=150)
                kv.reset(0)
                S.prefill(m, kv, 0, ids[:70], 0, logit_rows=0)
                part, tok2 = S.prefill(m, kv, 0, ids[70:], 70, logit_rows=80)
            finally:
                kv.close()
            runs[mode] = (full, tok, part, tok2)
        for mode in ("tiles", "mfma"):
            for i, what in ((0, "single prefill"), (2, "chunked prefill")):
                got, ref = runs[mode][i], runs["rows"][i]
                err = float(np.max(np.abs(got - ref)))
                assert err <= 1e-3 * float(np.max(np.abs(ref))), f"{mode}, {what}: max abs diff {err:.3e}"
            assert runs[mode][1] == runs["rows"][1] and runs[mode][3] == runs["rows"][3]
    finally:
        m.close()


@pytest.mark.parametrize("hilo", ["0", "1", "default", "o,down"])
@pytest.mark.parametrize("n", [150, 300, 2000])
def test_prefill_split_gemm_matches_staged_kernel(gpu_ctx, monkeypatch, n, hilo):
    """The prefill projections on fp16 activations written by their producers (RMSNorm, attention and the SwiGLU
    epilogue; direct-to-LDS pipeline) form the same products in the same order as the register-staged MFMA kernel
    that converts the fp32 activations itself, with hi/lo pairs on every projection (SOC_PREFILL_SPLIT=1), on none
    (0), on the QKV projection only (the default) and on another mix: logits are bit-identical, for a single prefill
    (row counts off the 64/128-row tiles) and a chunked one. Qwen3-0.6B-wide layers (hidden 1024, 16 q / 8 kv heads,
    3072). At 2000 rows the projections take the 8-wave tile configurations (128-row tiles; 256 x 192 for gate/up),
    the 77-row chunk the small ones."""
    if hilo == "default":
        monkeypatch.delenv("SOC_PREFILL_SPLIT", raising=False)
    else:
        monkeypatch.setenv("SOC_PREFILL_SPLIT", hilo)
    cfg = S.QwenConfig(vocab_size=512, hidden_size=1024, num_hidden_layers=2, num_attention_heads=16,
                       num_key_value_heads=8, intermediate_size=3072, tie_word_embeddings=True)
    m = _gpu_model(gpu_ctx, cfg, S.synth_weights(cfg, 21))
    ids = S.synth_tokens(22, "split", cfg.vocab_size, n)
    runs = {}
    try:
        for mode in ("staged", "split"):
            if mode == "staged":
                monkeypatch.setenv("SOC_PREFILL_GEMM", "staged")
            else:
                monkeypatch.delenv("SOC_PREFILL_GEMM", raising=False)
            kv = S.KVCache(m, 1, n + 8)
            try:
                full, tok = S.prefill(m, kv, 0, ids, 0, logit_rows=n)
                kv.reset(0)
                S.prefill(m, kv, 0, ids[:77], 0, logit_rows=0)
                part, tok2 = S.prefill(m, kv, 0, ids[77:], 77, logit_rows=n - 77)
            finally:
                kv.close()
            runs[mode] = (full, tok, part, tok2)
        for i in (0, 2):
            np.testing.assert_array_equal(runs["split"][i], runs["staged"][i])
        assert runs["split"][1] == runs["staged"][1] and runs["split"][3] == runs["staged"][3]
    finally:
        m.close()


def test_decode_steps_equal_decode_loop(gpu_ctx):
    cfg, seed, _, _ = SMALL_MODELS["tiny_untied"]
    m = _gpu_model(gpu_ctx, cfg, S.synth_weights(cfg, seed))
    ids = S.synth_tokens(8, "steps", cfg.vocab_size, 7)
    a = S.KVCache(m, 1, 48)
    b = S.KVCache(m, 2, 48)
    try:
        _, t0 = S.prefill(m, a, 0, ids)
        _, u0 = S.prefill(m, b, 1, ids)
        assert t0 == u0
        loop = [t0]
        for _ in range(20):
            loop.append(S.decode(m, a, 0, loop[-1], want_logits=False)[1])
        steps = S.decode_steps(m, b, 1, u0, 20)
        assert steps.tolist() == loop[1:]
        assert a.length(0) == b.length(1) == 27
    finally:
        a.close()
        b.close()
        m.close()


@pytest.mark.parametrize("name", ["tiny_untied", "tiny_g4", "tiny_kv8"])
def test_persistent_decode_matches_graph_decode(gpu_ctx, name, monkeypatch):
    """The one-launch decode steps (with attention blocks; for 8 KV heads also the XCD-partitioned one) and the
    per-op kernels (graph replay) agree on every step."""
    cfg, seed, _, _ = SMALL_MODELS[name]
    m = _gpu_model(gpu_ctx, cfg, S.synth_weights(cfg, seed))
    ids = S.synth_tokens(9, "paths", cfg.vocab_size, 13)
    modes = ("graph", "persistent", "xcd") if cfg.num_key_value_heads == 8 else ("graph", "persistent")
    runs = {}
    try:
        for mode in modes:
            monkeypatch.setenv("SOC_DECODE", mode)
            assert m.decode_path() == mode, f"SOC_DECODE={mode} fell back to {m.decode_path()}"
            kv = S.KVCache(m, 1, 300)
            _, t = S.prefill(m, kv, 0, ids)
            rows, toks = [], [t]
            for _ in range(12):
                lg, t = S.decode(m, kv, 0, toks[-1])
                rows.append(lg)
                toks.append(t)
            # long run on the device-resident token loop crosses the 256-key attention chunk boundary
            more = S.decode_steps(m, kv, 0, toks[-1], 270)
            kv.close()
            runs[mode] = (np.stack(rows), toks, more)
        for mode in modes[1:]:
            assert runs["graph"][1] == runs[mode][1], mode
            assert_logits_close(runs[mode][0], runs["graph"][0], f"{name} {mode} vs graph")
            assert np.array_equal(runs["graph"][2], runs[mode][2]), mode
    finally:
        m.close()


def test_prefill_against_live_oracle_long_prompt(gpu_ctx, oracle_mod):
    """Qwen3-0.6B layer shapes (4 of its 28 layers), 512-token prompt, last-row logits vs the oracle."""
    cfg = S.QwenConfig(vocab_size=151936, hidden_size=1024, num_hidden_layers=4, num_attention_heads=16,
                       num_key_value_heads=8, intermediate_size=3072)
    w = S.synth_weights(cfg, 3)
    ids = S.synth_tokens(3, "prompt", cfg.vocab_size, 512)
    m = _gpu_model(gpu_ctx, cfg, w)
    kv = S.KVCache(m, 1, 520)
    try:
        logits, tok = S.prefill(m, kv, 0, ids, 0, logit_rows=1)
        om = oracle_mod.OracleModel(cfg, w)
        cache = oracle_mod.OracleCache(om, 520)
        ref = cache.forward(ids, 0, logit_rows=1)
        assert_logits_close(logits[0], ref[0], "last row")
        assert tok == oracle_mod.sample(ref[0])
        # three decode steps after the long prompt
        t = tok
        for i in range(3):
            lg, nt = S.decode(m, kv, 0, t)
            r = cache.forward(np.array([t], np.int32), 512 + i)
            assert_logits_close(lg, r[0], f"decode {i}")
            assert nt == oracle_mod.sample(r[0])
            t = nt
    finally:
        kv.close()
        m.close()


@pytest.mark.parametrize("fixture", ["qwen3_0p6b.npz", "qwen3_0p6b_s2.npz"])
@pytest.mark.parametrize("mode", ["xcd", "persistent", "graph"])
def test_qwen3_0p6b_greedy_matches_reference(gpu_ctx, golden, mode, fixture, monkeypatch):
    """Qwen3-0.6B, random-init fp16 weights (seed 1, N(0, 0.02): one repeated token; seed 2, N(0, 0.05): 16 distinct
    tokens), 32-token prompt, 16 greedy tokens at batch 1 through each decode implementation: host-stepped soc_decode
    with per-step logit checks, then the device-fed loop soc_decode_steps (the benchmarked path) from a fresh cache."""
    g = golden(fixture)
    cfg = S.QWEN3_0_6B
    sigma = float(g["sigma"]) if "sigma" in g else 0.02
    monkeypatch.setenv("SOC_DECODE", mode)
    m = S.Model(gpu_ctx, cfg).synthesize(int(g["weight_seed"]), sigma)
    kv = S.KVCache(m, 1, 64)
    try:
        assert m.decode_path() == mode
        prompt = g["prompt"]
        logits, tok = S.prefill(m, kv, 0, prompt)
        rows = [logits[0]]
        toks = [tok]
        for _ in range(15):
            lg, tok = S.decode(m, kv, 0, toks[-1])
            rows.append(lg)
            toks.append(tok)
        assert toks == g["tokens"].tolist()
        for i, lg in enumerate(rows):
            assert_logits_close(lg[g["sample_idx"]], g["sample_vals"][i], f"{fixture} {mode} step {i} sampled")
            assert_logits_close(lg[g["top_ids"][i]], g["top_vals"][i], f"{fixture} {mode} step {i} top-64")
        kv.reset(0)
        _, first = S.prefill(m, kv, 0, prompt, 0, logit_rows=0)
        dev = S.decode_steps(m, kv, 0, first, 15)
        assert [first] + dev.tolist() == g["tokens"].tolist()
    finally:
        kv.close()
        m.close()


@pytest.mark.parametrize("nq,layers", [(8, 3), (16, 3), (16, 5)])
def test_xcd_decode_g1_and_odd_layers(gpu_ctx, nq, layers, monkeypatch):
    """The XCD-partitioned decode with one query head per KV head (8 q / 8 kv, the G = 1 kernel) and with odd layer
    counts (the exchange tags of a layer then differ in parity from step to step), at hidden 1024 / intermediate
    3072 (Qwen3-0.6B layer shapes), against the per-op graph path: host-stepped logits, then 300 device-fed steps
    that cross the split-attention thresholds at 257 and 289 keys."""
    cfg = S.QwenConfig(vocab_size=4096, hidden_size=1024, num_hidden_layers=layers, num_attention_heads=nq,
                       num_key_value_heads=8, intermediate_size=3072, tie_word_embeddings=False)
    m = S.Model(gpu_ctx, cfg).synthesize(11, 0.05)
    ids = S.synth_tokens(12, "xcd.g1", cfg.vocab_size, 9)
    runs = {}
    try:
        for mode in ("graph", "xcd"):
            monkeypatch.setenv("SOC_DECODE", mode)
            assert m.decode_path() == mode
            kv = S.KVCache(m, 1, 320)
            _, t = S.prefill(m, kv, 0, ids)
            rows, toks = [], [t]
            for _ in range(6):
                lg, t = S.decode(m, kv, 0, toks[-1])
                rows.append(lg)
                toks.append(t)
            more = S.decode_steps(m, kv, 0, toks[-1], 300)
            kv.close()
            runs[mode] = (np.stack(rows), toks, more)
        assert runs["graph"][1] == runs["xcd"][1]
        assert_logits_close(runs["xcd"][0], runs["graph"][0], f"nq {nq} L {layers} xcd vs graph")
        same = runs["graph"][2] == runs["xcd"][2]
        assert same.all(), f"first difference at device step {int(np.argmin(same))}"
    finally:
        m.close()


@pytest.mark.parametrize("mode", ["xcd", "persistent"])
def test_one_launch_wait_timeout_recovers(gpu_ctx, mode, monkeypatch):
    """A step whose cross-block wait timed out (forced from the host: the error flag is raised before the launches, so
    every block of every launch leaves at entry) fails the call with SOC_ERR_HIP and a time-out message, keeps the KV
    length, does not switch the model off the one-launch path (a time-out is not a placement failure), and the next
    call decodes exactly as the per-op path does."""
    cfg, seed, _, _ = SMALL_MODELS["tiny_kv8"]
    m = _gpu_model(gpu_ctx, cfg, S.synth_weights(cfg, seed))
    ids = S.synth_tokens(9, "paths", cfg.vocab_size, 13)
    try:
        monkeypatch.setenv("SOC_DECODE", "graph")
        kv = S.KVCache(m, 1, 64)
        _, t = S.prefill(m, kv, 0, ids)
        want = S.decode_steps(m, kv, 0, t, 8)
        kv.close()
        monkeypatch.setenv("SOC_DECODE", mode)
        assert m.decode_path() == mode
        kv = S.KVCache(m, 1, 64)
        _, t = S.prefill(m, kv, 0, ids)
        S.decode_steps(m, kv, 0, t, 2)  # exchange state initialised and in use
        kv.reset(0)
        _, t = S.prefill(m, kv, 0, ids)
        monkeypatch.setenv("SOC_FORCE_WAIT_ERROR", "1")
        with pytest.raises(S.SocError) as e:
            S.decode_steps(m, kv, 0, t, 4)
        assert e.value.code == S.capi.SOC_ERR_HIP
        assert "timed out" in str(e.value)
        assert kv.length(0) == len(ids)
        monkeypatch.delenv("SOC_FORCE_WAIT_ERROR")
        assert m.decode_path() == mode
        got = S.decode_steps(m, kv, 0, t, 8)
        assert np.array_equal(got, want)
        kv.close()
    finally:
        m.close()


@pytest.mark.parametrize("split", ["1", "0", "default"])
def test_prefill_2048_matches_reference(gpu_ctx, golden, split, monkeypatch):
    """The benchmarked prefill: Qwen3-0.6B (seed-1 weights), 2048 uniform-random prompt ids, all 28 layers; last-row
    logits (top 64, 512 sampled ids) and greedy token against the restatement's fixture (pinned bit for bit to the
    compiled reference at 256 tokens of the same model). split=1 feeds every projection hi/lo fp16 pairs, split=0
    single fp16 activations, the default hi/lo pairs on the QKV projection only; the errors are printed."""
    g = golden("prefill2048.npz")
    cfg = S.QWEN3_0_6B
    if split == "default":
        monkeypatch.delenv("SOC_PREFILL_SPLIT", raising=False)
    else:
        monkeypatch.setenv("SOC_PREFILL_SPLIT", split)
    m = S.Model(gpu_ctx, cfg).synthesize(int(g["weight_seed"]), 0.02)
    n = int(g["n"])
    kv = S.KVCache(m, 1, n)
    try:
        ids = S.synth_tokens(int(g["ids_seed"]), "prefill", cfg.vocab_size, n)
        logits, tok = S.prefill(m, kv, 0, ids)
        assert tok == int(g["argmax"])
        assert_logits_close(logits[0][g["top_ids"][0]], g["top_vals"][0], f"prefill 2048 split={split} top-64")
        assert_logits_close(logits[0][g["sample_idx"]], g["sample_vals"][0], f"prefill 2048 split={split} sampled")
    finally:
        kv.close()
        m.close()


def test_error_paths_leave_state_unchanged(gpu_ctx):
    """Host-forced failures (Mac/gpu/src/runtime/generation_context.cpp:22-27,67-90; kv_cache.mm:103-108)."""
    cfg, seed, _, _ = SMALL_MODELS["tiny_tied"]
    m = S.Model(gpu_ctx, cfg)
    kv = S.KVCache(m, 1, 16)
    try:
        with pytest.raises(S.SocError) as e:
            S.prefill(m, kv, 0, [1, 2, 3])
        assert e.value.code == S.capi.SOC_ERR_STATE  # not finalized
        m.load(S.synth_weights(cfg, seed))
        with pytest.raises(S.SocError) as e:
            S.prefill(m, kv, 0, np.zeros(0, np.int32))
        assert e.value.code == S.capi.SOC_ERR_INVALID
        with pytest.raises(S.SocError) as e:
            S.prefill(m, kv, 0, [1, cfg.vocab_size])
        assert e.value.code == S.capi.SOC_ERR_INVALID
        with pytest.raises(S.SocError) as e:
            S.prefill(m, kv, 0, np.arange(17, dtype=np.int32))
        assert e.value.code == S.capi.SOC_ERR_CAPACITY
        assert kv.length(0) == 0
        S.prefill(m, kv, 0, np.arange(15, dtype=np.int32))
        with pytest.raises(S.SocError) as e:
            S.prefill(m, kv, 0, [1], position_offset=3)
        assert e.value.code == S.capi.SOC_ERR_STATE
        _, t = S.decode(m, kv, 0, 1)
        with pytest.raises(S.SocError) as e:
            S.decode(m, kv, 0, t)
        assert e.value.code == S.capi.SOC_ERR_CAPACITY
        assert kv.length(0) == 16
        with pytest.raises(S.SocError) as e:
            S.decode(m, kv, 5, 1)
        assert e.value.code == S.capi.SOC_ERR_INVALID
        kv.reset(0)
        assert kv.length(0) == 0
        _, t2 = S.prefill(m, kv, 0, [3])
        assert kv.length(0) == 1
    finally:
        kv.close()
        m.close()
