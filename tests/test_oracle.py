"""Pins the CPU oracle (oracle/soc_oracle.cpp) before it is trusted as the checker.

Each function of the oracle is checked against (a) golden vectors written by the reference's own compiled sources
(tests/golden/*.npz, see make_golden.py), (b) the reference's known-answer tests re-derived here
(Mac/cpu/test/test_nn_modules.cpp), and (c) closed forms / invariants chosen so that a dropped term, a wrong sign or
index, or a transposed operand fails at least one of them.
"""
import math

import numpy as np
import pytest

from soc_amd import QwenConfig, synth_tokens, synth_weights


def f32(x):
    return np.float32(x)


# ---------------------------------------------------------------------------------------------------------------
# dtype (Mac/cpu/src/dtype.cpp:76-156)
# ---------------------------------------------------------------------------------------------------------------
def test_f16_to_f32_exhaustive(oracle_mod, golden):
    g = golden("dtype_f16.npz")
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle_mod.f16_to_f32(codes)
    # golden vector from the compiled reference, all 65,536 codes, bit for bit
    assert np.array_equal(got.view(np.uint32), g["f16_to_f32_bits"])
    # closed form: IEEE binary16 -> binary32 is exact; NaN payloads keep their bits shifted by 13
    want = codes.view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))


def test_f32_to_f16_matches_reference(oracle_mod, golden):
    g = golden("dtype_f16.npz")
    got = np.array([oracle_mod.f32_to_f16(float(x)) for x in g["f32_inputs"]], dtype=np.uint16)
    assert np.array_equal(got, g["f32_to_f16_bits"])
    # the reference rounds the magnitude half-up (not to even): 1 + 2^-11 lies halfway -> rounds up to 1 + 2^-10
    assert oracle_mod.f32_to_f16(1.00048828125) == 0x3C01
    assert oracle_mod.f32_to_f16(65504.0) == 0x7BFF and oracle_mod.f32_to_f16(1e6) == 0x7C00


# ---------------------------------------------------------------------------------------------------------------
# ops vs golden vectors of the compiled reference (bit-exact: same operation order)
# ---------------------------------------------------------------------------------------------------------------
def test_ops_match_reference_bitwise(oracle_mod, golden):
    g = golden("ops_small.npz")
    O = oracle_mod
    assert np.array_equal(O.linear_f16(g["linear_x"], g["linear_w"]), g["linear_y"])
    assert np.array_equal(O.rmsnorm_f16(g["rms_x"], g["rms_g"], 1e-6), g["rms_y"])
    assert np.array_equal(O.rope(g["rope_x"], 1e6, 1000), g["rope_y"])
    assert np.array_equal(O.gqa(g["gqa_q"], g["gqa_k"], g["gqa_v"], prefix=7), g["gqa_o"])
    picks = [O.sample(g["sample_row"], 1.0, k) for k in (1, 2, 3, 7)]
    assert picks == g["sample_picks"].tolist()
    picks2 = [O.sample(g["sample_row2"], t, k) for t, k in ((1.0, 1), (0.7, 5), (2.0, 50))]
    assert picks2 == g["sample_picks2"].tolist()


def test_ops_fixture_is_sensitive(oracle_mod, golden):
    """A wrong RoPE offset, a transposed weight or a missing causal mask would not match the golden vectors."""
    g = golden("ops_small.npz")
    O = oracle_mod
    assert not np.allclose(O.rope(g["rope_x"], 1e6, 1001), g["rope_y"], atol=1e-4)
    w = g["linear_w"]
    assert not np.allclose(O.linear_f16(g["linear_x"][:, :40], np.ascontiguousarray(w[:, :40].T)),
                           g["linear_y"][:, :40], atol=1e-3)
    assert not np.allclose(O.gqa(g["gqa_q"], g["gqa_k"], g["gqa_v"], prefix=7, causal=False), g["gqa_o"], atol=1e-4)


# ---------------------------------------------------------------------------------------------------------------
# Known-answer tests of Mac/cpu/test/test_nn_modules.cpp, re-derived
# ---------------------------------------------------------------------------------------------------------------
def test_kat_linear(oracle_mod):
    # test_nn_modules.cpp:106-137 (the reference adds a bias; Qwen3 projections have none, so compare x.W^T + b)
    w = np.array([[1.0, 2.0, 3.0], [-1.0, 0.5, 4.0]], dtype=np.float32)
    x = np.array([[1.0, 0.0, -1.0], [2.0, 1.0, 0.5]], dtype=np.float32)
    y = oracle_mod.linear_f32(x, w) + np.array([0.25, -0.5], dtype=np.float32)
    assert np.allclose(y, [[-1.75, -5.5], [5.75, 0.0]], atol=1e-5)


def test_kat_rmsnorm(oracle_mod):
    # test_nn_modules.cpp:157-186
    g = np.array([1.0, 1.5, 0.5], dtype=np.float32)
    x = np.array([[3.0, 4.0, 0.0], [1.0, 2.0, 2.0]], dtype=np.float32)
    y = oracle_mod.rmsnorm_f32(x, g, 1e-6)
    s0 = 1.0 / math.sqrt(25.0 / 3.0 + 1e-6)
    s1 = 1.0 / math.sqrt(9.0 / 3.0 + 1e-6)
    assert abs(y[0, 0] - 3 * s0) < 1e-5 and abs(y[0, 1] - 4 * s0 * 1.5) < 1e-5
    assert abs(y[1, 0] - s1) < 1e-5 and abs(y[1, 2] - 2 * s1 * 0.5) < 1e-5
    # invariant: with unit gain the output rms is 1 (up to eps)
    x = np.random.default_rng(0).normal(0, 3, (4, 128)).astype(np.float32)
    y = oracle_mod.rmsnorm_f32(x, np.ones(128, np.float32), 1e-6)
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(1)), 1.0, atol=1e-5)


def test_kat_rope(oracle_mod):
    # test_nn_modules.cpp:201-241: d=4, theta=1e4; position 0 is the identity; angles 1 and 0.01 at position 1
    x = np.array([[[1.0, 2.0, 10.0, 20.0]], [[3.0, 4.0, 30.0, 40.0]]], dtype=np.float32)
    y = oracle_mod.rope(x, 1e4, 0)
    assert np.allclose(y[0, 0], [1, 2, 10, 20], atol=1e-6)
    a0, a1 = 1.0, 0.01
    assert np.allclose(y[1, 0], [3 * math.cos(a0) - 30 * math.sin(a0), 4 * math.cos(a1) - 40 * math.sin(a1),
                                 3 * math.sin(a0) + 30 * math.cos(a0), 4 * math.sin(a1) + 40 * math.cos(a1)],
                       atol=1e-5)
    y = oracle_mod.rope(np.array([[[5.0, 6.0, 7.0, 8.0]]], np.float32), 1e4, 3)
    assert abs(y[0, 0, 0] - (5 * math.cos(3.0) - 7 * math.sin(3.0))) < 1e-5
    assert abs(y[0, 0, 1] - (6 * math.cos(0.03) - 8 * math.sin(0.03))) < 1e-5
    # invariant: rotation keeps each (i, i + d/2) pair's norm
    x = np.random.default_rng(1).normal(0, 1, (3, 2, 128)).astype(np.float32)
    y = oracle_mod.rope(x, 1e6, 77)
    n0 = x[..., :64] ** 2 + x[..., 64:] ** 2
    n1 = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)


def test_kat_gqa(oracle_mod):
    # test_nn_modules.cpp:252-310: 2 q heads share 1 kv head, d=2, causal
    q = np.array([[[1, 0], [0, 1]], [[0.5, 0.5], [1, 0]]], dtype=np.float32)
    k = np.array([[[1, 0]], [[0, 1]]], dtype=np.float32)
    v = np.array([[[10, 1]], [[2, 20]]], dtype=np.float32)
    o = oracle_mod.gqa(q, k, v)
    assert np.allclose(o[0, 0], [10, 1]) and np.allclose(o[0, 1], [10, 1])
    sc = 1 / math.sqrt(2)
    w0, w1 = math.exp(0.5 * sc - 0.5 * sc), math.exp(0.5 * sc - 0.5 * sc)
    assert np.allclose(o[1, 0], [(w0 * 10 + w1 * 2) / (w0 + w1), (w0 * 1 + w1 * 20) / (w0 + w1)], atol=1e-5)
    s10, s11 = 1 * sc, 0.0
    m = max(s10, s11)
    w0, w1 = math.exp(s10 - m), math.exp(s11 - m)
    assert np.allclose(o[1, 1], [(w0 * 10 + w1 * 2) / (w0 + w1), (w0 * 1 + w1 * 20) / (w0 + w1)], atol=1e-5)
    # special cases: one visible key -> v; all scores equal -> mean of v (brute force over a longer prefix)
    rng = np.random.default_rng(2)
    v = rng.normal(0, 1, (9, 1, 8)).astype(np.float32)
    kz = np.zeros((9, 1, 8), np.float32)
    qz = rng.normal(0, 1, (1, 2, 8)).astype(np.float32)
    o = oracle_mod.gqa(qz, kz, v, prefix=8)
    assert np.allclose(o[0, 0], v[:, 0].mean(0), atol=1e-6) and np.allclose(o[0, 1], v[:, 0].mean(0), atol=1e-6)
    o = oracle_mod.gqa(qz, kz[:1], v[:1], prefix=0)
    assert np.allclose(o[0, 0], v[0, 0])


def test_gqa_matches_float64_softmax(oracle_mod):
    rng = np.random.default_rng(3)
    T, S, nq, nkv, d, P = 4, 11, 6, 3, 32, 7
    q = rng.normal(0, 1, (T, nq, d)).astype(np.float32)
    k = rng.normal(0, 1, (S, nkv, d)).astype(np.float32)
    v = rng.normal(0, 1, (S, nkv, d)).astype(np.float32)
    o = oracle_mod.gqa(q, k, v, prefix=P)
    for t in range(T):
        for h in range(nq):
            g = h // (nq // nkv)
            vis = P + t + 1
            s = (k[:vis, g].astype(np.float64) @ q[t, h].astype(np.float64)) / math.sqrt(d)
            w = np.exp(s - s.max())
            w /= w.sum()
            assert np.allclose(o[t, h], w @ v[:vis, g].astype(np.float64), atol=2e-5)


def test_sample_topk_restatement(oracle_mod):
    """The GPU sampler's list: first id == sample() (pinned to the compiled reference), values the k largest of
    logit / t in order, top_k clamped to [1, vocab], non-positive temperature taken as 1."""
    rng = np.random.default_rng(5)
    for trial in range(200):
        v = int(rng.integers(1, 400))
        row = rng.integers(-3, 4, v).astype(np.float32) * np.float32(rng.choice([1.0, 0.37]))
        for k in (0, 1, 2, 5, 50, 1000):
            for t in (1.0, 0.7, 0.0, -1.0):
                tok, ids, vals = oracle_mod.sample_topk(row, t, k)
                kk = max(1, min(k, v))
                tt = np.float32(t if t > 0 else 1.0)
                assert ids.size == kk and tok == ids[0]
                assert tok == oracle_mod.sample(row, float(tt), kk)
                q = row[ids] / tt
                assert np.all(q[:-1] >= q[1:])
                assert np.array_equal(np.sort(row / tt)[::-1][:kk], q)
                assert np.array_equal(vals, row[ids])
                assert len(set(ids.tolist())) == kk


def test_kat_sampler(oracle_mod):
    # test_nn_modules.cpp:619-628
    assert oracle_mod.sample(np.array([0.1, 3.0, 2.0], np.float32), 1.0, 2) == 1
    # greedy ties resolve to the lowest index
    assert oracle_mod.sample(np.array([1.0, 5.0, 5.0, 5.0], np.float32), 1.0, 1) == 1


def _tiny_cfg(**kw):
    base = dict(vocab_size=4, hidden_size=4, num_hidden_layers=1, num_attention_heads=1, num_key_value_heads=1,
                intermediate_size=4, head_dim=4, max_position_embeddings=16)
    base.update(kw)
    return QwenConfig(**base)


def _f16(a):
    return np.asarray(a, dtype=np.float16).view(np.uint16)


def test_kat_identity_model_generation(oracle_mod):
    """Mac/gpu/test/runtime/test_generation_context.mm:35-140: identity embedding, zero projections -> [2,2,2]."""
    cfg = _tiny_cfg()
    eye = np.eye(4, dtype=np.float32)
    z = np.zeros((4, 4), np.float32)
    one = np.ones(4, np.float32)
    p = "model.layers.0."
    w = {"model.embed_tokens.weight": _f16(eye), "model.norm.weight": _f16(one),
         p + "input_layernorm.weight": _f16(one), p + "post_attention_layernorm.weight": _f16(one),
         p + "self_attn.q_norm.weight": _f16(one), p + "self_attn.k_norm.weight": _f16(one)}
    for n in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
              "mlp.up_proj", "mlp.down_proj"):
        w[p + n + ".weight"] = _f16(z)
    m = oracle_mod.OracleModel(cfg, w)
    toks, _ = m.generate(np.array([1, 2], np.int32), 3, max_seq=8, top_k=2)
    assert toks.tolist() == [2, 2, 2]
    # zero block = identity residual (test_nn_modules.cpp:476-508): logits = 2 * e_token . E^T
    logits = m.forward_logits(np.array([0, 3], np.int32))
    assert np.allclose(logits, 2 * eye[[0, 3]], atol=1e-5)


def _small_model(oracle_mod, tied=False, seed=4):
    cfg = QwenConfig(vocab_size=300, hidden_size=128, num_hidden_layers=2, num_attention_heads=2,
                     num_key_value_heads=1, intermediate_size=256, tie_word_embeddings=tied)
    return cfg, oracle_mod.OracleModel(cfg, synth_weights(cfg, seed))


def test_cached_equals_uncached(oracle_mod):
    """test_nn_modules.cpp:358-403 and :535-591: cached decode reproduces the full forward's rows bit for bit."""
    cfg, m = _small_model(oracle_mod)
    ids = synth_tokens(4, "prompt", cfg.vocab_size, 10)
    full = m.forward_logits(ids)
    cache = oracle_mod.OracleCache(m, 16)
    first = cache.forward(ids[:6], 0, logit_rows=6)
    assert np.array_equal(first, full[:6])
    for t in range(6, 10):
        row = cache.forward(ids[t:t + 1], t)
        assert np.array_equal(row[0], full[t])
    assert cache.length() == 10


def test_small_models_match_reference(oracle_mod, golden):
    from tests.golden.make_golden import SMALL_MODELS

    for name, (cfg, seed, plen, new) in SMALL_MODELS.items():
        g = golden(f"model_{name}.npz")
        w = synth_weights(cfg, seed)
        prompt = synth_tokens(seed, "prompt", cfg.vocab_size, plen)
        assert np.array_equal(prompt, g["prompt"]), "generator changed: fixtures are stale"
        m = oracle_mod.OracleModel(cfg, w)
        toks, logits = m.generate(prompt, new, want_logits=True)
        assert np.array_equal(toks, g["tokens"]), name
        assert np.array_equal(logits, g["step_logits"]), name
        assert np.array_equal(m.forward_logits(prompt), g["prompt_logits"]), name


def test_quant_int8_percol_matches_reference(oracle_mod, golden):
    g = golden("quant_int8.npz")
    codes, scales = oracle_mod.quant_int8_percol(g["rhs"])
    assert np.array_equal(codes, g["codes"]) and np.array_equal(scales, g["scales"])
    y = oracle_mod.matmul_quant_int8(g["a"], codes, scales)
    assert np.array_equal(y, g["y"])
    assert np.all(y[:, 5] == 0.0) and scales[5] == 0.0


def test_group_quant_closed_form(oracle_mod):
    """The group-64 int8/int4 format: dequant is exact (w = code * scale), and the matmul follows from it."""
    rng = np.random.default_rng(6)
    N, K = 24, 256
    for bits in (8, 4):
        if bits == 8:
            codes = rng.integers(-128, 128, (N, K)).astype(np.int8)
            cint = codes.astype(np.int64)
            packed = codes
        else:
            cint = rng.integers(-8, 8, (N, K)).astype(np.int64)
            nib = (cint & 0xF).astype(np.uint8)
            packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
        scales = rng.uniform(0.005, 0.02, (N, K // 64)).astype(np.float16)
        w = oracle_mod.dequant_group(packed, bits, scales, N, K)
        want = cint.astype(np.float64) * np.repeat(scales.astype(np.float64), 64, axis=1)
        assert np.array_equal(w.astype(np.float64), want)  # exact: products fit in fp32
        a = rng.normal(0, 1, (3, K)).astype(np.float16)
        y = oracle_mod.qmm_group(a, packed, bits, scales, K, N)
        ref = a.astype(np.float64) @ want.T
        assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)
        # a nibble-order or scale-index mistake would break this: swap the nibbles / shift the groups
        if bits == 4:
            swapped = ((packed >> 4) | (packed << 4)).astype(np.uint8)
            assert not np.allclose(oracle_mod.qmm_group(a, swapped, bits, scales, K, N), ref, atol=1e-3)
        shifted = np.roll(scales, 1, axis=1)
        assert not np.allclose(oracle_mod.qmm_group(a, packed, bits, shifted, K, N), ref, atol=1e-3)


def test_group_quant_equal_scales_reduce_to_int_matmul(oracle_mod):
    rng = np.random.default_rng(8)
    N, K = 16, 192
    codes = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s = np.float16(0.0125)
    scales = np.full((N, K // 64), s, np.float16)
    a = rng.normal(0, 1, (2, K)).astype(np.float16)
    y = oracle_mod.qmm_group(a, codes, 8, scales, K, N)
    ref = (a.astype(np.float64) @ codes.astype(np.float64).T) * float(s)
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.skipif(not __import__("oracle.oracle", fromlist=["ref_available"]).ref_available(),
                    reason="reference library not built here")
def test_port_matches_compiled_reference_random_model(oracle_mod):
    """Where oracle/_ref exists: port and reference agree bit for bit on a fresh random model and prompt."""
    cfg, m = _small_model(oracle_mod, tied=False, seed=21)
    w = synth_weights(cfg, 21)
    r = oracle_mod.OracleModel(cfg, w, "reference")
    ids = synth_tokens(21, "prompt", cfg.vocab_size, 7)
    tp, lp = m.generate(ids, 5, want_logits=True)
    tr, lr = r.generate(ids, 5, want_logits=True)
    assert np.array_equal(tp, tr) and np.array_equal(lp, lr)
