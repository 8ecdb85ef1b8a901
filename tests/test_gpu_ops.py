"""Op-level parity on the GPU: every entry point of the C ABI that runs one piece of the forward on caller memory, and
the forward in each of the reference's forms (QwenCausalLM::Forward{Hidden,Logits}[Cached], qwen_causal_lm.cpp:37-268).

* soc_forward uncached (kv = NULL) against the oracle's uncached forward (forward_logits with a position offset),
  all rows, on every small model including eight query heads per KV head; uncached logits equal the cached forward's
  from an empty cache bit for bit; hidden rows times the head equal the logits; device token ids give the same bits
  as host ids, and an out-of-range id in device memory fails the call without advancing the cache.
* soc_gemm_f16 (the prefill projection GEMM) at 2048 rows on every Qwen3-0.6B projection shape against the oracle's
  Linear (linear.cpp:51-84) on the same fp16-rounded activations.
* soc_attention_prefill at 2048 x 2048 with 16 query / 8 KV heads (and a chunk at a prefix), and 8 query heads on
  one KV head, against the oracle's GroupedQueryAttention (grouped_query_attention.cpp:59-142).
* soc_attention_decode over 1 .. 4096 keys for 1, 2, 4 and 8 query heads per KV head against the same oracle.
* The reference's fp32 op kernels (soc_op_*: MatMul with bias / residual / SiLU / transposed rhs, RMSNorm, RoPE,
  Softmax, Embedding, ElementwiseMul) against the oracle where it has the op (linear_f32, rmsnorm_f32, rope) and the
  closed form elsewhere (float64 numpy).
"""
import ctypes as C

import numpy as np
import pytest

import soc_amd as S
from tests.golden.make_golden import SMALL_MODELS
from tests.parity import assert_logits_close

pytestmark = pytest.mark.gpu

L = S.lib


def _assert_close(got, ref, atol, what):
    err = float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))))
    print(f"[parity] {what}: max abs err {err:.3e} (tol {atol:g})", flush=True)
    assert err <= atol, f"{what}: max abs err {err:.3e} > {atol:g}"


# ---- the forward in the reference's forms ----

@pytest.mark.parametrize("name", list(SMALL_MODELS))
@pytest.mark.parametrize("offset", [0, 7])
def test_uncached_forward_matches_oracle(gpu_ctx, oracle_mod, name, offset):
    cfg, seed, plen, _ = SMALL_MODELS[name]
    w = S.synth_weights(cfg, seed)
    ids = S.synth_tokens(seed, "prompt", cfg.vocab_size, plen)
    ref = oracle_mod.OracleModel(cfg, w).forward_logits(ids, offset)
    m = S.Model(gpu_ctx, cfg).load(w)
    try:
        hidden, logits, tok = S.forward(m, None, 0, ids, offset, want_hidden=True, logit_rows=plen)
        assert_logits_close(logits, ref, f"{name} uncached forward at offset {offset}, all {plen} rows")
        assert tok == int(np.argmax(logits[-1]))
        # ComputeLogitsFromHidden (qwen_causal_lm.cpp:270-300): the hidden rows through the head give the logits
        head = w["model.embed_tokens.weight" if cfg.tie_word_embeddings else "lm_head.weight"]
        head = head.view(np.float16).astype(np.float64)
        assert_logits_close(hidden.astype(np.float64) @ head.T, ref, f"{name} hidden rows x head")
        # the private cache is left empty: a second call gives the same bits
        h2, l2, _ = S.forward(m, None, 0, ids, offset, want_hidden=True, logit_rows=plen)
        assert np.array_equal(l2, logits) and np.array_equal(h2, hidden)
    finally:
        m.close()


@pytest.mark.parametrize("name", ["tiny_untied", "tiny_g8", "tiny_kv8"])
def test_forward_logits_equal_cached_forward(gpu_ctx, name):
    """Uncached at offset 0 and cached from an empty cache run the same kernels on the same inputs: equal bits, for
    the logits and the hidden rows."""
    cfg, seed, plen, _ = SMALL_MODELS[name]
    w = S.synth_weights(cfg, seed)
    ids = S.synth_tokens(seed + 1, "forward", cfg.vocab_size, plen)
    m = S.Model(gpu_ctx, cfg).load(w)
    kv = S.KVCache(m, 2, 64)
    try:
        hu, lu, tu = S.forward(m, None, 0, ids, 0, want_hidden=True, logit_rows=plen)
        hc, lc, tc = S.forward(m, kv, 1, ids, 0, want_hidden=True, logit_rows=plen)
        assert np.array_equal(lu, lc) and np.array_equal(hu, hc) and tu == tc
        assert kv.length(1) == plen and kv.length(0) == 0
        # and the cached forward's decode step matches the prefill of the whole sequence's last row
        _, ld, _ = S.forward(m, kv, 1, [tc], plen, logit_rows=1)
        _, lall, _ = S.forward(m, None, 0, np.append(ids, tc), 0, logit_rows=1)
        assert_logits_close(ld[0], lall[0], f"{name} cached decode vs uncached prefill of the sequence")
    finally:
        kv.close()
        m.close()


@pytest.mark.parametrize("name", ["tiny_tied", "tiny_kv8"])
def test_forward_device_token_ids(gpu_ctx, name):
    """Token ids in device memory: the same bits as host ids on the prefill and the decode path; an id outside the
    vocabulary fails the call after it ran, the slot length stays, and the next call is unaffected."""
    cfg, seed, plen, _ = SMALL_MODELS[name]
    w = S.synth_weights(cfg, seed)
    ids = S.synth_tokens(seed, "prompt", cfg.vocab_size, plen)
    m = S.Model(gpu_ctx, cfg).load(w)
    kv = S.KVCache(m, 2, 64)
    dev = gpu_ctx.upload(np.append(ids, [0, cfg.vocab_size]).astype(np.int32))
    try:
        _, lh, th = S.forward(m, kv, 0, ids, 0, logit_rows=2)
        _, ld, td = S.forward(m, kv, 1, ids, 0, logit_rows=2, ids_dev=dev)
        assert np.array_equal(lh, ld) and th == td
        nxt = np.array([th], np.int32)
        gpu_ctx.write(dev + 4 * plen, nxt)
        _, lh1, th1 = S.forward(m, kv, 0, nxt, plen, logit_rows=1)
        _, ld1, td1 = S.forward(m, kv, 1, nxt, plen, logit_rows=1, ids_dev=dev + 4 * plen)
        assert np.array_equal(lh1, ld1) and th1 == td1
        assert kv.length(0) == kv.length(1) == plen + 1
        with pytest.raises(S.SocError, match="token id out of range"):
            S.forward(m, kv, 1, np.zeros(1, np.int32), plen + 1, logit_rows=1, ids_dev=dev + 4 * (plen + 1))
        assert kv.length(1) == plen + 1
        with pytest.raises(S.SocError, match="token id out of range"):
            S.forward(m, None, 0, np.zeros(2, np.int32), 0, logit_rows=1, ids_dev=dev + 4 * plen)
        _, ld2, _ = S.forward(m, kv, 1, nxt, plen + 1, logit_rows=1, ids_dev=dev + 4 * plen)
        _, lh2, _ = S.forward(m, kv, 0, nxt, plen + 1, logit_rows=1)
        assert np.array_equal(lh2, ld2)
    finally:
        gpu_ctx.free(dev)
        kv.close()
        m.close()


# ---- the prefill projection GEMM ----

@pytest.mark.parametrize("shape", [("qkv", 4096, 1024), ("q_proj", 2048, 1024), ("k_proj/v_proj", 1024, 1024),
                                   ("o_proj", 1024, 2048), ("gate/up_proj", 3072, 1024), ("down_proj", 1024, 3072)])
def test_gemm_f16_prefill_shapes(gpu_ctx, oracle_mod, shape):
    what, n, k = shape
    m_rows = 2048
    rng = np.random.default_rng(n + k)
    x = rng.standard_normal((m_rows, k)).astype(np.float16)
    wt = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    ref = oracle_mod.linear_f16(x.astype(np.float32), wt.view(np.uint16))
    px, pw, py = gpu_ctx.upload(x), gpu_ctx.upload(wt), gpu_ctx.alloc(m_rows * n * 4)
    try:
        S.gemm_f16(gpu_ctx, px, pw, py, m_rows, n, k)
        y = gpu_ctx.download(py, (m_rows, n), np.float32)
    finally:
        for p in (px, pw, py):
            gpu_ctx.free(p)
    # fp16 products are exact in fp32; only the summation order differs from Linear's ascending loop
    _assert_close(y, ref, 2e-5 * np.sqrt(k) * float(np.max(np.abs(ref))) + 1e-5, f"gemm {what} {m_rows}x{n}x{k}")


def test_gemm_f16_ragged_shapes_and_bad_operands(gpu_ctx, oracle_mod):
    rng = np.random.default_rng(3)
    for m_rows, n, k in ((1, 96, 64), (37, 200, 160), (130, 1000, 96)):
        x = rng.standard_normal((m_rows, k)).astype(np.float16)
        wt = (rng.standard_normal((n, k)) * 0.05).astype(np.float16)
        px, pw, py = gpu_ctx.upload(x), gpu_ctx.upload(wt), gpu_ctx.alloc(m_rows * n * 4)
        try:
            S.gemm_f16(gpu_ctx, px, pw, py, m_rows, n, k)
            y = gpu_ctx.download(py, (m_rows, n), np.float32)
            with pytest.raises(S.SocError, match="past the end"):
                S.gemm_f16(gpu_ctx, px, pw, py, m_rows + 1, n, k)
        finally:
            for p in (px, pw, py):
                gpu_ctx.free(p)
        _assert_close(y, oracle_mod.linear_f16(x.astype(np.float32), wt.view(np.uint16)), 1e-4, f"gemm {m_rows}x{n}x{k}")
    with pytest.raises(S.SocError, match="multiple of 32"):
        S.gemm_f16(gpu_ctx, 0, 0, 0, 4, 4, 40)
    host = np.zeros(64 * 64, np.float16)
    with pytest.raises(S.SocError, match="not in device memory"):
        S.gemm_f16(gpu_ctx, host.ctypes.data, host.ctypes.data, host.ctypes.data, 2, 2, 32)


# ---- attention ----

def _kv_planes(rng, nkv, cap):
    k = rng.standard_normal((nkv, cap, 128)).astype(np.float16)
    v = rng.standard_normal((nkv, cap, 128)).astype(np.float16)
    return k, v


def _oracle_attn(oracle_mod, q, k, v, s_len, prefix):
    kf = np.ascontiguousarray(k[:, :s_len].astype(np.float32).transpose(1, 0, 2))
    vf = np.ascontiguousarray(v[:, :s_len].astype(np.float32).transpose(1, 0, 2))
    return oracle_mod.gqa(q, kf, vf, prefix=prefix, causal=True)


@pytest.mark.parametrize("heads,rows,pos_base", [((16, 8), 2048, 0), ((16, 8), 256, 1792), ((32, 8), 300, 77),
                                                 ((8, 1), 512, 0), ((8, 8), 200, 50)])
def test_attention_prefill_matches_oracle(gpu_ctx, oracle_mod, heads, rows, pos_base):
    nq, nkv = heads
    cap = pos_base + rows
    rng = np.random.default_rng(nq * 7 + rows)
    # q as the model feeds it: RMS-normed heads (|q| ~ sqrt(128)) times the 1/sqrt(d) the kernel applies
    q = rng.standard_normal((rows, nq, 128)).astype(np.float32)
    k, v = _kv_planes(rng, nkv, cap)
    ref = _oracle_attn(oracle_mod, q, k, v, cap, pos_base)
    pq, pk, pv, po = gpu_ctx.upload(q), gpu_ctx.upload(k), gpu_ctx.upload(v), gpu_ctx.alloc(q.nbytes)
    try:
        S.attention_prefill(gpu_ctx, pq, pk, pv, po, rows, pos_base, nq, nkv, cap)
        out = gpu_ctx.download(po, q.shape, np.float32)
    finally:
        for p in (pq, pk, pv, po):
            gpu_ctx.free(p)
    _assert_close(out, ref, 3e-3, f"prefill attention {nq}q/{nkv}kv rows {rows} at {pos_base}")


@pytest.mark.parametrize("heads", [(16, 8), (32, 8), (8, 1), (8, 8)])
def test_attention_decode_matches_oracle(gpu_ctx, oracle_mod, heads):
    nq, nkv = heads
    cap = 4096
    rng = np.random.default_rng(nq + 3 * nkv)
    k, v = _kv_planes(rng, nkv, cap)
    pk, pv = gpu_ctx.upload(k), gpu_ctx.upload(v)
    pq, po = gpu_ctx.alloc(nq * 128 * 4), gpu_ctx.alloc(nq * 128 * 4)
    try:
        for s_len in (1, 2, 100, 256, 257, 1000, 2049, 4096):
            q = rng.standard_normal((1, nq, 128)).astype(np.float32)
            gpu_ctx.write(pq, q)
            S.attention_decode(gpu_ctx, pq, pk, pv, po, s_len, nq, nkv, cap)
            out = gpu_ctx.download(po, q.shape, np.float32)
            ref = _oracle_attn(oracle_mod, q, k, v, s_len, s_len - 1)
            _assert_close(out, ref, 2e-3, f"decode attention {nq}q/{nkv}kv over {s_len} keys")
        with pytest.raises(S.SocError, match="kv_len"):
            S.attention_decode(gpu_ctx, pq, pk, pv, po, cap + 1, nq, nkv, cap)
    finally:
        for p in (pk, pv, pq, po):
            gpu_ctx.free(p)


# ---- the reference's fp32 op kernels ----

def _run(ctx, fn, *args):
    rc = fn(ctx.h, *args)
    if rc != 0:
        raise S.SocError(rc, L().soc_last_error().decode())


def test_op_matmul_forms(gpu_ctx, oracle_mod):
    rng = np.random.default_rng(5)
    for rows, inner, cols in ((1, 64, 64), (3, 100, 37), (70, 130, 129), (256, 512, 96)):
        lhs = rng.standard_normal((rows, inner)).astype(np.float32)
        rhs = rng.standard_normal((inner, cols)).astype(np.float32)
        bias = rng.standard_normal(cols).astype(np.float32)
        res = rng.standard_normal((rows, cols)).astype(np.float32)
        exact = lhs.astype(np.float64) @ rhs.astype(np.float64)
        # Linear (linear_f32: y = x . W^T with W [out][in]) is the transposed-rhs form
        lin = oracle_mod.linear_f32(lhs, np.ascontiguousarray(rhs.T))
        tol = 4e-6 * np.sqrt(inner) * float(np.max(np.abs(exact))) + 1e-6
        pl, pr, prt = gpu_ctx.upload(lhs), gpu_ctx.upload(rhs), gpu_ctx.upload(np.ascontiguousarray(rhs.T))
        pb, pres, po = gpu_ctx.upload(bias), gpu_ctx.upload(res), gpu_ctx.alloc(rows * cols * 4)
        try:
            _run(gpu_ctx, L().soc_op_matmul, pl, pr, None, None, po, rows, inner, cols, 0, 0)
            _assert_close(gpu_ctx.download(po, (rows, cols), np.float32), exact, tol, f"matmul {rows}x{inner}x{cols}")
            _run(gpu_ctx, L().soc_op_matmul, pl, prt, None, None, po, rows, inner, cols, 1, 0)
            _assert_close(gpu_ctx.download(po, (rows, cols), np.float32), lin, tol, f"matmul transposed vs Linear")
            # bias, residual (aliasing the output), SiLU: (x W + b + r) / (1 + exp(-(...))) (gpu_kernels.metal:276-284)
            gpu_ctx.write(po, res)
            _run(gpu_ctx, L().soc_op_matmul, pl, pr, pb, po, po, rows, inner, cols, 0, 1)
            z = exact + bias + res
            _assert_close(gpu_ctx.download(po, (rows, cols), np.float32), z / (1 + np.exp(-z)), tol + 1e-6,
                          "matmul bias + residual + SiLU")
        finally:
            for p in (pl, pr, prt, pb, pres, po):
                gpu_ctx.free(p)
    host = np.zeros(16, np.float32)
    with pytest.raises(S.SocError, match="not in device memory"):
        _run(gpu_ctx, L().soc_op_matmul, host.ctypes.data, host.ctypes.data, None, None, host.ctypes.data, 2, 2, 2, 0, 0)


def test_op_rmsnorm_rope_softmax_mul(gpu_ctx, oracle_mod):
    rng = np.random.default_rng(9)
    rows, heads, d = 7, 4, 128
    x = rng.standard_normal((rows, heads * d)).astype(np.float32) * 3
    gain = rng.uniform(0.5, 1.5, heads * d).astype(np.float32)
    px, pg, py = gpu_ctx.upload(x), gpu_ctx.upload(gain), gpu_ctx.alloc(x.nbytes)
    try:
        _run(gpu_ctx, L().soc_op_rmsnorm, px, pg, py, rows, heads * d, C.c_float(1e-6))
        _assert_close(gpu_ctx.download(py, x.shape, np.float32), oracle_mod.rmsnorm_f32(x, gain, 1e-6), 2e-6,
                      "rmsnorm")
        for off in (0, 5, 4000):
            _run(gpu_ctx, L().soc_op_rope, px, py, rows, heads, d, d, off, C.c_double(1e6))
            ref = oracle_mod.rope(x.reshape(rows, heads, d), 1e6, off).reshape(rows, heads * d)
            _assert_close(gpu_ctx.download(py, x.shape, np.float32), ref, 1e-6, f"rope at offset {off}")
        # partial rotary (rope_op.mm: rotary_dim < head_dim): the first 64 dims rotate with exponent 2i / 64, the
        # rest pass through; in place
        gpu_ctx.write(py, x)
        _run(gpu_ctx, L().soc_op_rope, py, py, rows, heads, d, 64, 3, C.c_double(1e4))
        got = gpu_ctx.download(py, x.shape, np.float32).reshape(rows, heads, d)
        xr = x.reshape(rows, heads, d).astype(np.float64)
        i = np.arange(32)
        ang = (3 + np.arange(rows))[:, None] / np.power(1e4, 2 * i / 64)[None, :]
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        want = xr.copy()
        want[..., :32] = xr[..., :32] * c - xr[..., 32:64] * s
        want[..., 32:64] = xr[..., :32] * s + xr[..., 32:64] * c
        _assert_close(got, want, 2e-5, "partial rotary, in place")
        _run(gpu_ctx, L().soc_op_softmax, px, py, rows, heads * d)
        e = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True))
        _assert_close(gpu_ctx.download(py, x.shape, np.float32), e / e.sum(axis=1, keepdims=True), 1e-7, "softmax")
        _run(gpu_ctx, L().soc_op_mul, px, pg, py, 1, heads * d)
        got = gpu_ctx.download(py, (heads * d,), np.float32)
        assert np.array_equal(got, x[0] * gain)
    finally:
        for p in (px, pg, py):
            gpu_ctx.free(p)


def test_op_embedding(gpu_ctx):
    rng = np.random.default_rng(2)
    vocab, hidden = 50, 96
    ids = np.array([0, 49, 7, -1, 50, 3], np.int32)
    for dt, code in ((np.float32, 0), (np.float16, 1)):
        table = rng.standard_normal((vocab, hidden)).astype(dt)
        pi, pt, po = gpu_ctx.upload(ids), gpu_ctx.upload(table), gpu_ctx.alloc(ids.size * hidden * 4)
        try:
            _run(gpu_ctx, L().soc_op_embedding, pi, pt, code, po, ids.size, hidden, vocab)
            got = gpu_ctx.download(po, (ids.size, hidden), np.float32)
        finally:
            for p in (pi, pt, po):
                gpu_ctx.free(p)
        want = np.zeros((ids.size, hidden), np.float32)
        for r, t in enumerate(ids):
            if 0 <= t < vocab:
                want[r] = table[t].astype(np.float32)
        assert np.array_equal(got, want)  # out-of-range ids give zero rows (gpu_kernels.metal:114-117)
