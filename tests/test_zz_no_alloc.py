"""soc_decode_steps_noalloc (device buffers from the library's static scratch array, no allocation) against
soc_decode_steps on the same inputs: identical tokens and identical KV cache contents, for two calls in a row, the
second with a smaller input, on each one-launch decode kernel; sizes beyond the array are rejected."""
import numpy as np
import pytest

import soc_amd as S
from tests.golden.make_golden import SMALL_MODELS

pytestmark = pytest.mark.gpu


def _kv_bytes(kv, m):
    return [kv.read(0, layer) for layer in range(m.cfg.num_hidden_layers)]


@pytest.mark.parametrize("mode,name", [("xcd", "tiny_kv8"), ("persistent", "tiny_g4")])
def test_noalloc_steps_equal_decode_steps(gpu_ctx, mode, name, monkeypatch):
    cfg, seed, _, _ = SMALL_MODELS[name]
    monkeypatch.setenv("SOC_DECODE", mode)
    m = S.Model(gpu_ctx, cfg).load(S.synth_weights(cfg, seed))
    try:
        assert m.decode_path() == mode
        # call 1: 13-token prompt, 300 steps (crosses the 256-key attention split); call 2: 4-token prompt, 9 steps
        for plen, steps in ((13, 300), (4, 9)):
            ids = S.synth_tokens(40 + plen, "noalloc", cfg.vocab_size, plen)
            a = S.KVCache(m, 1, 320)
            b = S.KVCache(m, 1, 320)
            try:
                _, ta = S.prefill(m, a, 0, ids)
                _, tb = S.prefill(m, b, 0, ids)
                assert ta == tb
                want = S.decode_steps(m, a, 0, ta, steps)
                got = S.decode_steps_noalloc(m, b, 0, tb, steps)
                print(f"[noalloc] {mode} {name} prompt {plen} steps {steps}: tokens equal "
                      f"{bool(np.array_equal(got, want))}", flush=True)
                assert np.array_equal(got, want)
                assert a.length(0) == b.length(0) == plen + steps
                for (ka, va), (kb, vb) in zip(_kv_bytes(a, m), _kv_bytes(b, m)):
                    assert np.array_equal(ka.view(np.uint16), kb.view(np.uint16))
                    assert np.array_equal(va.view(np.uint16), vb.view(np.uint16))
            finally:
                a.close()
                b.close()
    finally:
        m.close()


def test_noalloc_rejects_sizes_beyond_scratch(gpu_ctx, monkeypatch):
    cfg, seed, _, _ = SMALL_MODELS["tiny_kv8"]
    monkeypatch.setenv("SOC_DECODE", "xcd")
    m = S.Model(gpu_ctx, cfg).load(S.synth_weights(cfg, seed))
    kv = S.KVCache(m, 1, 16)
    try:
        _, t = S.prefill(m, kv, 0, [1, 2, 3])
        with pytest.raises(S.SocError) as e:
            S.decode_steps_noalloc(m, kv, 0, t, 2_000_000)
        assert e.value.code == S.capi.SOC_ERR_CAPACITY
        assert "scratch" in str(e.value)
        assert kv.length(0) == 3
        got = S.decode_steps_noalloc(m, kv, 0, t, 5)
        assert got.shape == (5,) and kv.length(0) == 8
    finally:
        kv.close()
        m.close()
