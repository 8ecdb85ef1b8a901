"""Bundle reading without a GPU (soc_bundle_*): the reference loader test (Mac/cpu/test/test_model_loader.cpp:80-155)
on bundles written here, in float32 and in float16 with bfloat16 gains; conversions to the fp16 the model keeps;
and the validation messages of startup_validator.cpp:5-23, qwen3_config.cpp:42-67, weight_loader.cpp:17-30 and
qwen_model_loader.cpp:17-25."""
import numpy as np
import pytest

import soc_amd as S
from tests.bundle import config_dict, f32_to_bf16_bits, write_bundle

TINY = S.QwenConfig(vocab_size=2, hidden_size=2, num_hidden_layers=1, num_attention_heads=1, num_key_value_heads=1,
                    intermediate_size=2, head_dim=2, rope_theta=10000.0, tie_word_embeddings=True)


def _loader_tensors(export_dtype):
    """test_model_loader.cpp:80-118: identity embedding, unit gains, zero projections."""
    gain_dtype = "float32" if export_dtype == "float32" else "bfloat16"
    w_dtype = export_dtype
    eye = np.array([[1.0, 0.0], [0.0, 1.0]], np.float32)
    z = np.zeros((2, 2), np.float32)
    one = np.ones(2, np.float32)
    p = "model.layers.0."
    return {
        "model.embed_tokens.weight": (eye, w_dtype),
        p + "input_layernorm.weight": (one, gain_dtype),
        p + "self_attn.q_proj.weight": (z, w_dtype), p + "self_attn.k_proj.weight": (z, w_dtype),
        p + "self_attn.v_proj.weight": (z, w_dtype), p + "self_attn.o_proj.weight": (z, w_dtype),
        p + "self_attn.q_norm.weight": (np.ones(2, np.float32), gain_dtype),
        p + "self_attn.k_norm.weight": (np.ones(2, np.float32), gain_dtype),
        p + "post_attention_layernorm.weight": (one, gain_dtype),
        p + "mlp.gate_proj.weight": (z, w_dtype), p + "mlp.up_proj.weight": (z, w_dtype),
        p + "mlp.down_proj.weight": (z, w_dtype),
        "model.norm.weight": (one, gain_dtype),
    }


@pytest.mark.parametrize("export_dtype", ["float32", "float16"])
def test_model_loader_smoke(tmp_path, oracle_mod, export_dtype):
    path = write_bundle(tmp_path, config_dict(TINY, export_dtype), _loader_tensors(export_dtype),
                        export_dtype=export_dtype)
    b = S.Bundle(path)
    cfg = b.config()
    assert cfg.hidden_size == 2 and cfg.vocab_size == 2 and cfg.tie_word_embeddings
    w = {name: b.tensor_f16(name, shape) for name, shape in S.tensor_specs(cfg)}
    b.close()
    assert np.array_equal(w["model.embed_tokens.weight"].view(np.float16), np.eye(2, dtype=np.float16))
    # the reference test's forward over tokens [0, 1] (test_model_loader.cpp:140-147), on the oracle
    om = oracle_mod.OracleModel(cfg, w)
    logits = om.forward_logits(np.array([0, 1], np.int32))
    assert logits.shape == (2, 2)
    assert logits[0, 0] > logits[0, 1], "token 0 hidden state should favor vocab row 0 under tied embeddings"
    assert logits[1, 1] > logits[1, 0], "token 1 hidden state should favor vocab row 1 under tied embeddings"


def test_dtype_conversions_round_to_nearest_even(tmp_path):
    rng = np.random.default_rng(4)
    vals = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 3,
                           np.array([65504.0, 65519.0, 1e-8, -0.0, 2.0 ** -24, 3 * 2.0 ** -25], np.float32)])
    n = vals.size
    cfg = S.QwenConfig(vocab_size=n // 2, hidden_size=2, num_hidden_layers=1, num_attention_heads=1,
                       num_key_value_heads=1, intermediate_size=2, head_dim=2, tie_word_embeddings=True)
    for dtype in ("float32", "bfloat16", "float16"):
        t = _loader_tensors("float32")
        # the largest values stay finite after the source dtype's own rounding (bfloat16 rounds 65504 up to 65536)
        if dtype == "bfloat16":
            vals[-6:-4] = 65280.0
        t["model.embed_tokens.weight"] = (vals.reshape(n // 2, 2), dtype)
        with np.errstate(over="ignore"):
            path = write_bundle(tmp_path / dtype, config_dict(cfg), t)
        b = S.Bundle(path)
        got = b.tensor_f16("model.embed_tokens.weight", (n // 2, 2)).reshape(-1)
        b.close()
        src = vals if dtype != "bfloat16" else (f32_to_bf16_bits(vals).astype(np.uint32) << 16).view(np.float32)
        want = src.astype(np.float16).view(np.uint16)  # numpy: IEEE round to nearest even
        assert np.array_equal(got, want), dtype


def test_weights_beyond_fp16_range_are_refused(tmp_path):
    """The device keeps fp16: a finite float32 / bfloat16 weight that rounds to inf in fp16 (|w| >= 65520) is an error
    naming the tensor, while 65504 (fp16's largest finite value) and non-finite source values load as they are."""
    cfg = S.QwenConfig(vocab_size=4, hidden_size=2, num_hidden_layers=1, num_attention_heads=1,
                       num_key_value_heads=1, intermediate_size=2, head_dim=2, tie_word_embeddings=True)
    for dtype, bad in (("float32", 65520.0), ("float32", -1e6), ("bfloat16", 70000.0)):
        t = _loader_tensors("float32")
        t["model.embed_tokens.weight"] = (np.array([[1.0, 2.0], [3.0, bad], [0, 0], [0, 0]], np.float32), dtype)
        path = write_bundle(tmp_path / f"{dtype}_{bad}", config_dict(cfg), t)
        b = S.Bundle(path)
        with pytest.raises(S.SocError, match="outside the float16 range.*model.embed_tokens.weight"):
            b.tensor_f16("model.embed_tokens.weight", (4, 2))
        b.close()
    t = _loader_tensors("float32")
    t["model.embed_tokens.weight"] = (np.array([[65504.0, -65504.0], [np.inf, -np.inf], [0, 0], [0, 0]], np.float32),
                                      "float32")
    b = S.Bundle(write_bundle(tmp_path / "edge", config_dict(cfg), t))
    got = b.tensor_f16("model.embed_tokens.weight", (4, 2)).reshape(-1)
    b.close()
    assert got[:4].tolist() == [0x7BFF, 0xFBFF, 0x7C00, 0xFC00]


def _expect_error(path, text):
    with pytest.raises(S.SocError) as e:
        b = S.Bundle(path)
        cfg = b.config()
        for name, shape in S.tensor_specs(cfg):
            b.tensor_f16(name, shape)
    assert text in str(e.value), str(e.value)


def test_validation_messages(tmp_path):
    base = _loader_tensors("float32")
    cfg = config_dict(TINY, "float32")
    cases = [
        (dict(manifest_overrides={"format": "other"}), "manifest format must be soc.cpp.llm_export"),
        (dict(manifest_overrides={"format_version": 1}), "manifest format_version must be at least 2"),
        (dict(manifest_overrides={"config": []}), "manifest config must be a JSON object"),
        (dict(manifest_overrides={"tensors": []}), "manifest must contain at least one tensor"),
        (dict(drop=("tokenizer_runtime_file",)), "manifest must reference tokenizer_runtime_file"),
        (dict(byte_size_delta={"model.norm.weight": 4}),
         "tensor record byte_size does not match dtype and shape for: model.norm.weight"),
        (dict(truncate={"model.layers.0.mlp.up_proj.weight": 8}),
         "tensor file is smaller than expected byte_size for: model.layers.0.mlp.up_proj.weight"),
    ]
    for i, (kw, text) in enumerate(cases):
        _expect_error(write_bundle(tmp_path / f"c{i}", cfg, base, **kw), text)
    bad = dict(base)
    bad["model.layers.0.self_attn.q_proj.weight"] = (np.zeros((2, 2), np.int32), "int32")
    _expect_error(write_bundle(tmp_path / "int", cfg, bad),
                  "model loader requires floating-point weights for: model.layers.0.self_attn.q_proj.weight")
    bad = dict(base)
    bad["model.norm.weight"] = (np.ones(3, np.float32), "float32")
    _expect_error(write_bundle(tmp_path / "shape", cfg, bad),
                  "model loader encountered unexpected shape for: model.norm.weight")
    bad = dict(base)
    del bad["model.layers.0.mlp.down_proj.weight"]
    _expect_error(write_bundle(tmp_path / "missing", cfg, bad),
                  "missing tensor in manifest: model.layers.0.mlp.down_proj.weight")
    for key, val, text in [("model_type", "llama", "config model_type must be qwen3"),
                           ("num_key_value_heads", 0, "qwen3 attention dimensions must be non-zero"),
                           ("rope_theta", 0, "qwen3 normalization and rope parameters must be positive"),
                           ("torch_dtype", "", "torch_dtype must not be empty")]:
        c2 = dict(cfg)
        c2[key] = val
        _expect_error(write_bundle(tmp_path / f"cfg_{key}", c2, base), text)
    c2 = dict(cfg)
    del c2["head_dim"]
    _expect_error(write_bundle(tmp_path / "nohd", c2, base), "missing JSON object key: head_dim")
    (tmp_path / "broken").mkdir()
    (tmp_path / "broken" / "manifest.json").write_text('{"format": "soc.cpp.llm_export", ')
    _expect_error(tmp_path / "broken" / "manifest.json", "unexpected end of JSON input")
    _expect_error(tmp_path / "nowhere" / "manifest.json", "failed to open JSON file")


def test_untied_requires_lm_head_and_max_positions_default(tmp_path):
    cfg = S.QwenConfig(vocab_size=2, hidden_size=2, num_hidden_layers=1, num_attention_heads=1, num_key_value_heads=1,
                       intermediate_size=2, head_dim=2, tie_word_embeddings=False)
    c = config_dict(cfg)
    del c["max_position_embeddings"]
    path = write_bundle(tmp_path, c, _loader_tensors("float32"))
    b = S.Bundle(path)
    assert b.config().max_position_embeddings == 32768
    _expect_error(path, "missing tensor in manifest: lm_head.weight")
