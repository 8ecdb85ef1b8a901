"""Ragged multi-sequence decode (soc_decode_batch / soc_decode_batch_steps) on an MI355X.

A batch row has the reference's one-sequence decode semantics for its own KV slot (GenerationContext::
DecodeNextToken, Mac/gpu/src/runtime/generation_context.cpp:68-172). Checks:
  (1) each row vs soc_decode of the same slot on an identical cache: logits within the model tolerance
      (max |diff| <= 2e-2 and <= 1e-2 * max |logit|), identical greedy tokens;
  (2) permuting the rows permutes the results bit for bit (rows are independent);
  (3) each row vs the CPU oracle's cached forward of that sequence, with KV lengths that mix short prefixes and
      several 256-key attention chunks;
  (4) soc_decode_batch_steps equals a loop of soc_decode_batch, bit for bit;
  (5) bad batches are rejected without touching any slot.
"""
import numpy as np
import pytest

import soc_amd as S
from tests.parity import assert_logits_close

pytestmark = pytest.mark.gpu

def small_cfg(nq=4, nkv=2):
    return S.QwenConfig(vocab_size=2048, hidden_size=256, num_hidden_layers=2, num_attention_heads=nq,
                        num_key_value_heads=nkv, intermediate_size=512, tie_word_embeddings=False)


PROMPT_LENS = [5, 17, 33, 2, 64]


def _prefilled_caches(m, cfg, count, cap=128):
    """`count` caches holding the same five prompts (GPU prefill) in slots 0..4; returns caches and last tokens."""
    caches, last = [], None
    for _ in range(count):
        kv = S.KVCache(m, len(PROMPT_LENS), cap)
        toks = []
        for slot, n in enumerate(PROMPT_LENS):
            ids = S.synth_tokens(20 + slot, "batch.prompt", cfg.vocab_size, n)
            _, t = S.prefill(m, kv, slot, ids, 0, logit_rows=0)
            toks.append(t)
        caches.append(kv)
        last = toks
    return caches, np.array(last, np.int32)


@pytest.mark.parametrize("nq,nkv", [(4, 2), (8, 2)])
def test_batch_rows_equal_single_sequence_decode(gpu_ctx, nq, nkv):
    cfg = small_cfg(nq, nkv)
    m = S.Model(gpu_ctx, cfg).load(S.synth_weights(cfg, 31))
    (a, b), last = _prefilled_caches(m, cfg, 2)
    try:
        order = np.array([3, 0, 4, 1, 2], np.int32)
        lg, nxt = S.decode_batch(m, a, order, last[order])
        for i, slot in enumerate(order):
            ref, t = S.decode(m, b, int(slot), int(last[slot]))
            assert_logits_close(lg[i], ref, f"row {i} (slot {slot})")
            assert int(nxt[i]) == t
            assert a.length(int(slot)) == b.length(int(slot)) == PROMPT_LENS[slot] + 1
    finally:
        a.close()
        b.close()
        m.close()


def test_batch_many_rows_slabs_and_tiled_path(gpu_ctx):
    """20 rows (two 16-row slabs of the skinny projection) and 70 rows (the tiled GEMM on the same pre-split
    activations): every row agrees with single-sequence decode of its slot within the model tolerance, with the
    same greedy token."""
    cfg = small_cfg()
    m = S.Model(gpu_ctx, cfg).load(S.synth_weights(cfg, 33))
    nslots = 70
    kvs = [S.KVCache(m, nslots, 32) for _ in range(2)]
    try:
        last = np.zeros(nslots, np.int32)
        for kv in kvs:
            for slot in range(nslots):
                ids = S.synth_tokens(40 + slot, "batch.many", cfg.vocab_size, 1 + slot % 7)
                _, last[slot] = S.prefill(m, kv, slot, ids, 0, logit_rows=0)
        for n in (20, 70):
            slots = np.arange(n, dtype=np.int32)[::-1].copy()
            lg, nxt = S.decode_batch(m, kvs[0], slots, last[slots])
            for i, slot in enumerate(slots):
                ref, t = S.decode(m, kvs[1], int(slot), int(last[slot]))
                assert_logits_close(lg[i], ref, f"{n} rows, row {i} (slot {slot})")
                assert int(nxt[i]) == t
            last[slots] = nxt
    finally:
        for kv in kvs:
            kv.close()
        m.close()


def test_batch_permutation_invariance_and_steps(gpu_ctx):
    cfg = small_cfg()
    m = S.Model(gpu_ctx, cfg).load(S.synth_weights(cfg, 32))
    (a, b), last = _prefilled_caches(m, cfg, 2)
    try:
        p1 = np.array([0, 1, 2, 3, 4], np.int32)
        p2 = np.array([4, 2, 0, 3, 1], np.int32)
        l1, n1 = S.decode_batch(m, a, p1, last[p1])
        l2, n2 = S.decode_batch(m, b, p2, last[p2])
        inv = np.argsort(p2)
        assert np.array_equal(l1, l2[inv]) and np.array_equal(n1, n2[inv])
        for slot in range(5):  # the appended keys/values agree too
            ka, va = a.read(slot, 1)
            kb, vb = b.read(slot, 1)
            assert np.array_equal(ka, kb) and np.array_equal(va, vb)
        # 4 graph-replayed steps == 4 single steps
        steps = S.decode_batch_steps(m, a, p1, n1, 4)
        tok, loop = n1.copy(), []
        for _ in range(4):
            _, tok = S.decode_batch(m, b, p1, tok)
            loop.append(tok.copy())
        assert np.array_equal(steps, np.stack(loop))
        for slot in range(5):
            assert a.length(slot) == b.length(slot) == PROMPT_LENS[slot] + 5
    finally:
        a.close()
        b.close()
        m.close()


def test_batch_matches_oracle_mixed_lengths(gpu_ctx, oracle_mod):
    """KV prefixes of 300, 5, 520 and 64 positions (seeded N(0,1) fp16 contents) in one batch: each row's logits
    and greedy token against the oracle's cached forward over the same (fp16-valued) prefix."""
    cfg = small_cfg()
    w = S.synth_weights(cfg, 33)
    m = S.Model(gpu_ctx, cfg).load(w)
    lens = [300, 5, 520, 64]
    kv = S.KVCache(m, len(lens), 544)
    try:
        for slot, n in enumerate(lens):
            kv.fill_synthetic(slot, n, 900 + slot)
        prefixes = {slot: [kv.read(slot, layer) for layer in range(cfg.num_hidden_layers)] for slot in range(4)}
        tokens = S.synth_tokens(34, "batch.tok", cfg.vocab_size, 4)
        slots = np.array([2, 0, 3, 1], np.int32)
        lg, nxt = S.decode_batch(m, kv, slots, tokens[slots])
        om = oracle_mod.OracleModel(cfg, w)
        for i, slot in enumerate(slots):
            n = lens[slot]
            cache = oracle_mod.OracleCache(om, n + 1)
            for layer, (k, v) in enumerate(prefixes[int(slot)]):
                for pos in range(n):
                    cache.write(layer, pos, k[:, pos, :].astype(np.float32), v[:, pos, :].astype(np.float32))
            ref = cache.forward(np.array([tokens[slot]], np.int32), n)
            assert_logits_close(lg[i], ref[0], f"row {i} (slot {slot}, {n} cached positions)")
            assert int(nxt[i]) == oracle_mod.sample(ref[0])
            assert kv.length(int(slot)) == n + 1
    finally:
        kv.close()
        m.close()


def test_ragged_qwen3_4b_matches_reference(gpu_ctx, golden):
    """The benchmarked ragged step at its own workload: Qwen3-4B (seed-1 weights), 16 sequences with KV lengths
    U[64, 4096] (seed 5) of seeded N(0, 1) fp16 contents, one token each (seed 6). The rows of the longest and
    shortest sequences and of slots 0 and 1 against the compiled reference's cached forward over the same caches;
    then a second step of all 16 rows, whose checked rows equal single-sequence decode of those slots."""
    g = golden("ragged4b.npz")
    cfg = S.QWEN3_4B
    m = S.Model(gpu_ctx, cfg).synthesize(int(g["weight_seed"]), 0.02)
    lens = g["kv_lens"].astype(np.int64)
    n = len(lens)
    kv = S.KVCache(m, n, int(lens.max()) + 4)
    try:
        for slot, ln in enumerate(lens):
            kv.fill_synthetic(slot, int(ln), 7)
        slots = np.arange(n, dtype=np.int32)
        toks = g["tokens"]
        lg, nxt = S.decode_batch(m, kv, slots, toks)
        for r, slot in enumerate(g["slots"]):
            what = f"4B ragged slot {int(slot)} (kv {int(lens[slot])})"
            assert int(nxt[slot]) == int(g["argmax"][r]), what
            assert_logits_close(lg[slot][g["top_ids"][r]], g["top_vals"][r], what + " top-64")
            assert_logits_close(lg[slot][g["sample_idx"]], g["sample_vals"][r], what + " sampled")
        # a second batch step vs one-sequence decode of the same slots (a second cache with the same contents in
        # those slots)
        lg2, nxt2 = S.decode_batch(m, kv, slots, nxt)
        one = S.KVCache(m, n, int(lens.max()) + 4)
        try:
            for slot in g["slots"]:
                slot = int(slot)
                one.fill_synthetic(slot, int(lens[slot]), 7)
                _, t0 = S.decode(m, one, slot, int(toks[slot]))
                assert t0 == int(nxt[slot])
                lg1, t1 = S.decode(m, one, slot, t0)
                assert t1 == int(nxt2[slot])
                assert_logits_close(lg2[slot], lg1, f"4B ragged slot {slot} batch step 2 vs decode")
        finally:
            one.close()
    finally:
        kv.close()
        m.close()


@pytest.mark.parametrize("pattern", ["repeated_rows", "all_zero"])
def test_batch_greedy_ties_across_chunks(gpu_ctx, pattern):
    """Exact ties in the greedy choice: a 65536-token LM head whose rows from 40000 on repeat 8 seeded rows (every
    maximum recurs ~3000 times, across all the blocks that scan a row), or an all-zero LM head (every logit 0).
    Each row's token must be the lowest index of its maximum logit: the reference's greedy pick
    (Mac/cpu/src/sampler.cpp:41-58, a top-1 partial sort, which replaces its candidate only on a strictly greater
    score)."""
    cfg = S.QwenConfig(vocab_size=65536, hidden_size=256, num_hidden_layers=2, num_attention_heads=4,
                       num_key_value_heads=2, intermediate_size=512, tie_word_embeddings=False)
    w = S.synth_weights(cfg, 36)
    head = np.zeros((cfg.vocab_size, cfg.hidden_size), np.float16)
    if pattern == "repeated_rows":
        rows = w["lm_head.weight"][:8]
        head[40000:] = rows[np.arange(cfg.vocab_size - 40000) % 8]
    w["lm_head.weight"] = head
    m = S.Model(gpu_ctx, cfg).load(w)
    (kv,), last = _prefilled_caches(m, cfg, 1)
    try:
        for n in (5, 1, 3):  # 64 blocks per row for each n
            slots = np.arange(n, dtype=np.int32)
            lg, nxt = S.decode_batch(m, kv, slots, last[slots])
            for i in range(n):
                want = int(np.argmax(lg[i]))  # numpy: first index of the maximum
                assert int(nxt[i]) == want, (pattern, n, i)
                if pattern == "all_zero":
                    assert want == 0
                else:
                    assert want >= 40000 or lg[i].max() == 0.0
            last[slots] = nxt
    finally:
        kv.close()
        m.close()


def test_batch_error_paths(gpu_ctx):
    cfg = small_cfg()
    m = S.Model(gpu_ctx, cfg).load(S.synth_weights(cfg, 35))
    kv = S.KVCache(m, 3, 8)
    try:
        for slot in range(3):
            S.prefill(m, kv, slot, np.array([1, 2, 3], np.int32), 0, logit_rows=0)
        with pytest.raises(S.SocError) as e:
            S.decode_batch(m, kv, [0, 0], [1, 2])  # duplicate slot
        assert e.value.code == S.capi.SOC_ERR_INVALID
        with pytest.raises(S.SocError) as e:
            S.decode_batch(m, kv, [0, 5], [1, 2])  # slot out of range
        assert e.value.code == S.capi.SOC_ERR_INVALID
        with pytest.raises(S.SocError) as e:
            S.decode_batch(m, kv, [0, 1], [1, cfg.vocab_size])  # token out of range
        assert e.value.code == S.capi.SOC_ERR_INVALID
        with pytest.raises(S.SocError) as e:
            S.decode_batch_steps(m, kv, [0, 1], [1, 2], 6)  # 3 + 6 > capacity 8
        assert e.value.code == S.capi.SOC_ERR_CAPACITY
        assert [kv.length(s) for s in range(3)] == [3, 3, 3]
        S.decode_batch_steps(m, kv, [2, 0], [1, 2], 5)
        assert [kv.length(s) for s in range(3)] == [8, 3, 8]
    finally:
        kv.close()
        m.close()
