"""On-device top-k sampling (soc_sample_topk) against the reference GPU sampler's result (oracle sample_topk: the
same std::partial_sort, Mac/gpu/src/runtime/sampler.cpp:44-66): identical token, candidate ids in the same order
(ties included) and raw logits, on rows with many ties, at the vocabulary size of Qwen3 and at small sizes, for
k in {1, 2, 5, 50, 64} (device search) and 65, 300 (host sort of the whole row); rows where every candidate
enters, where each chunk ascends, and rows longer than the device search takes at k = 64."""
import numpy as np
import pytest

import soc_amd as S

pytestmark = pytest.mark.gpu


def _rows():
    rng = np.random.default_rng(7)
    yield "qwen vocab, 9 distinct values", rng.integers(-4, 5, 151936).astype(np.float32)
    yield "qwen vocab, normal", rng.standard_normal(151936).astype(np.float32) * 3
    yield "ascending (every candidate enters)", np.arange(20000, dtype=np.float32)
    yield "ascending, 3000 candidates (more than the first readback holds)", np.arange(3000, dtype=np.float32)
    yield "ascending inside each 2048-chunk, descending across chunks", \
        np.concatenate([np.arange(2048, dtype=np.float32) - 3000 * c for c in range(6)])
    yield "saw tooth", np.tile(np.arange(300, dtype=np.float32), 40)
    yield "vocab 250000, normal", rng.standard_normal(250000).astype(np.float32)
    yield "descending", -np.arange(5000, dtype=np.float32)
    yield "all equal", np.zeros(4097, np.float32)
    yield "tiny", np.array([1.0, 5.0, 5.0, 5.0, -np.inf, 5.0, 2.0], np.float32)
    yield "with -inf and +-0", rng.choice(np.array([-np.inf, -0.0, 0.0, 1.0, 2.0], np.float32), 3000)


@pytest.mark.parametrize("k", [1, 2, 5, 50, 64, 65, 300])
@pytest.mark.parametrize("temperature", [1.0, 0.7, 0.0])
def test_sample_topk_matches_reference(gpu_ctx, oracle_mod, k, temperature):
    for what, row in _rows():
        p = gpu_ctx.upload(row)
        try:
            tok, ids, vals = S.sample_topk(gpu_ctx, p, row.size, k, temperature)
        finally:
            gpu_ctx.free(p)
        rtok, rids, rvals = oracle_mod.sample_topk(row, temperature, k)
        assert tok == rtok, what
        assert np.array_equal(ids, rids), f"{what}: first difference at rank {int(np.argmin(ids == rids))}"
        assert np.array_equal(vals.view(np.uint32), rvals.view(np.uint32)), what
        if temperature > 0:
            assert tok == oracle_mod.sample(row, temperature, k), what


def test_sample_topk_row_too_long_for_device_lists(gpu_ctx, oracle_mod):
    """400000 logits at k = 64: the per-chunk lists one block would merge exceed its LDS bound, so the row is sorted
    on the host; k = 5 on the same row stays on the device. Both equal the reference."""
    row = np.random.default_rng(5).standard_normal(400000).astype(np.float32)
    p = gpu_ctx.upload(row)
    try:
        for k in (5, 64):
            tok, ids, vals = S.sample_topk(gpu_ctx, p, row.size, k, 1.0)
            rtok, rids, rvals = oracle_mod.sample_topk(row, 1.0, k)
            assert tok == rtok and np.array_equal(ids, rids)
            assert np.array_equal(vals.view(np.uint32), rvals.view(np.uint32))
    finally:
        gpu_ctx.free(p)


def test_sample_topk_row_with_nan_uses_whole_row(gpu_ctx, oracle_mod):
    row = np.random.default_rng(3).standard_normal(10000).astype(np.float32)
    row[[5, 777]] = np.nan
    p = gpu_ctx.upload(row)
    try:
        for k in (1, 5):
            tok, ids, vals = S.sample_topk(gpu_ctx, p, row.size, k, 1.0)
            rtok, rids, _ = oracle_mod.sample_topk(row, 1.0, k)
            assert tok == rtok and np.array_equal(ids, rids)
    finally:
        gpu_ctx.free(p)


def test_sample_topk_on_decode_logits(gpu_ctx, oracle_mod):
    """Rows the model produced: the sampler on the device logits equals the oracle on their host copy."""
    from tests.golden.make_golden import SMALL_MODELS
    cfg, seed, _, _ = SMALL_MODELS["tiny_untied"]
    m = S.Model(gpu_ctx, cfg).load(S.synth_weights(cfg, seed))
    kv = S.KVCache(m, 1, 64)
    p = gpu_ctx.alloc(cfg.vocab_size * 4)
    try:
        lg, t = S.prefill(m, kv, 0, S.synth_tokens(3, "sampler", cfg.vocab_size, 9))
        for _ in range(4):
            lg, t = S.decode(m, kv, 0, t)
            gpu_ctx.write(p, lg)
            for k in (1, 5, 50):
                tok, ids, _ = S.sample_topk(gpu_ctx, p, cfg.vocab_size, k, 0.8)
                rtok, rids, _ = oracle_mod.sample_topk(lg, 0.8, k)
                assert tok == rtok and np.array_equal(ids, rids)
    finally:
        gpu_ctx.free(p)
        kv.close()
        m.close()


def test_sample_topk_row_in_pageable_host_memory(gpu_ctx, oracle_mod):
    """A row in pageable host memory (a numpy array) is classified before any launch and sorted on the host: same
    results as the device search and the reference, for k on both sides of the device limit."""
    row = np.random.default_rng(11).integers(-6, 7, 151936).astype(np.float32)
    p = gpu_ctx.upload(row)
    try:
        for k in (1, 5, 64, 65):
            dtok, dids, dvals = S.sample_topk(gpu_ctx, p, row.size, k, 0.9)
            htok, hids, hvals = S.sample_topk(gpu_ctx, row.ctypes.data, row.size, k, 0.9)
            rtok, rids, rvals = oracle_mod.sample_topk(row, 0.9, k)
            assert htok == dtok == rtok
            assert np.array_equal(hids, rids) and np.array_equal(dids, rids)
            assert np.array_equal(hvals.view(np.uint32), rvals.view(np.uint32))
    finally:
        gpu_ctx.free(p)


def test_sample_topk_rejects_row_past_its_allocation(gpu_ctx):
    """A device row shorter than `vocab` is refused on the host (checked against its allocation's extent)."""
    p = gpu_ctx.alloc(1000 * 4)
    try:
        with pytest.raises(S.SocError, match="past the end of its device allocation"):
            S.sample_topk(gpu_ctx, p, 1_000_000, 5, 1.0)
    finally:
        gpu_ctx.free(p)
