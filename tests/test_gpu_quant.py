"""Group-quantized models (soc_model_quantize) on the GPU against the oracle run on the same weights: the projections
packed by the library's packer and dequantized (w = code * scale, exact in fp32), everything else as the fp16 model.
Prefill logits of every row, greedy decode steps, and the device-fed decode loop; int8 and int4. A prompt of up to 8
rows runs the group-quantized kernels (exact products); a longer one the fp16 prefill kernels on each layer's
projections dequantized to fp16 (rounded to nearest). The GPU rounds the projections' input activations to fp16;
the tolerance is the model tolerance."""
import numpy as np
import pytest

import soc_amd as S
from tests.parity import assert_logits_close

pytestmark = pytest.mark.gpu

CFG = S.QwenConfig(vocab_size=1024, hidden_size=256, num_hidden_layers=2, num_attention_heads=4,
                   num_key_value_heads=2, intermediate_size=512, tie_word_embeddings=False)


def _dequantized(oracle_mod, w, bits):
    """The model's weights with every projection replaced by its dequantized group-quantized copy (fp32)."""
    out = dict(w)
    for name, arr in w.items():
        if any(p in name for p in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")):
            n, k = arr.shape
            codes, scales = S.quantize_group(arr, bits)
            out[name] = oracle_mod.dequant_group(codes, bits, scales, n, k)
    return out


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("n", [5, 13, 100])
def test_quantized_model_matches_oracle(gpu_ctx, oracle_mod, bits, n):
    w = S.synth_weights(CFG, 41, 0.05)
    m = S.Model(gpu_ctx, CFG).load(w).quantize(bits)
    om = oracle_mod.OracleModel(CFG, _dequantized(oracle_mod, w, bits))
    cap = n + 16
    kv = S.KVCache(m, 1, cap)
    try:
        assert m.decode_path() == "graph"
        ids = S.synth_tokens(42, "quant", CFG.vocab_size, n)
        lg, tok = S.prefill(m, kv, 0, ids, 0, logit_rows=n)
        cache = oracle_mod.OracleCache(om, cap)
        ref = cache.forward(ids, 0, logit_rows=n)
        assert_logits_close(lg, ref, f"int{bits} prefill rows, {n} tokens")
        assert tok == oracle_mod.sample(ref[-1])
        toks = [tok]
        for i in range(6):
            lg, t = S.decode(m, kv, 0, toks[-1])
            r = cache.forward(np.array([toks[-1]], np.int32), n + i)
            assert_logits_close(lg, r[0], f"int{bits} decode {i}")
            assert t == oracle_mod.sample(r[0])
            toks.append(t)
        # the device-fed loop (captured decode graph) from the same state
        kv2 = S.KVCache(m, 1, cap)
        try:
            _, t0 = S.prefill(m, kv2, 0, ids, 0, logit_rows=0)
            assert [t0] + S.decode_steps(m, kv2, 0, t0, 6).tolist() == toks
        finally:
            kv2.close()
        with pytest.raises(S.SocError):
            S.decode_batch(m, kv, [0], [toks[-1]])
        with pytest.raises(S.SocError):
            m.quantize(bits)  # already quantized
    finally:
        kv.close()
        m.close()
