"""ctypes binding of the C ABI declared in include/soc_hip.h (libsoc_hip.so, built in-tree).

This is the harness-side view of the boundary that tests and bench.py drive. Every non-zero status raises
SocError carrying the library's message. Loading fails loudly when the library has not been built.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libsoc_hip.so"

SOC_OK, SOC_ERR_INVALID, SOC_ERR_STATE, SOC_ERR_CAPACITY, SOC_ERR_HIP, SOC_ERR_NOMEM = range(6)


class SocError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[soc status {code}] {msg}")
        self.code = code


class QwenConfigC(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_int32), ("hidden_size", C.c_int32), ("num_hidden_layers", C.c_int32),
        ("num_attention_heads", C.c_int32), ("num_key_value_heads", C.c_int32), ("head_dim", C.c_int32),
        ("intermediate_size", C.c_int32), ("max_position_embeddings", C.c_int32), ("rope_theta", C.c_double),
        ("rms_norm_eps", C.c_float), ("tie_word_embeddings", C.c_int32),
    ]


@dataclass(frozen=True)
class QwenConfig:
    """Model hyper-parameters (the keys of the bundle's HF config, Mac/cpu/src/qwen3_config.cpp:20-36)."""
    vocab_size: int
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    intermediate_size: int
    head_dim: int = 128
    max_position_embeddings: int = 40960
    rope_theta: float = 1_000_000.0
    rms_norm_eps: float = 1e-6
    tie_word_embeddings: bool = True

    def to_c(self) -> QwenConfigC:
        return QwenConfigC(self.vocab_size, self.hidden_size, self.num_hidden_layers, self.num_attention_heads,
                           self.num_key_value_heads, self.head_dim, self.intermediate_size,
                           self.max_position_embeddings, self.rope_theta, self.rms_norm_eps,
                           1 if self.tie_word_embeddings else 0)

    @property
    def q_dim(self) -> int:
        return self.num_attention_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.num_key_value_heads * self.head_dim


# Dense Qwen3 shapes within this build's envelope (Hugging Face config.json of each model); 0.6B and 4B are the
# benchmarked ones.
QWEN3_0_6B = QwenConfig(vocab_size=151936, hidden_size=1024, num_hidden_layers=28, num_attention_heads=16,
                        num_key_value_heads=8, intermediate_size=3072)
QWEN3_1_7B = QwenConfig(vocab_size=151936, hidden_size=2048, num_hidden_layers=28, num_attention_heads=16,
                        num_key_value_heads=8, intermediate_size=6144)
QWEN3_4B = QwenConfig(vocab_size=151936, hidden_size=2560, num_hidden_layers=36, num_attention_heads=32,
                      num_key_value_heads=8, intermediate_size=9728)
QWEN3_8B = QwenConfig(vocab_size=151936, hidden_size=4096, num_hidden_layers=36, num_attention_heads=32,
                      num_key_value_heads=8, intermediate_size=12288, tie_word_embeddings=False)


def tensor_specs(cfg: QwenConfig) -> list[tuple[str, tuple[int, ...]]]:
    """Hugging Face tensor names and shapes (Mac/cpu/src/qwen_model_loader.cpp:43-92)."""
    H, I, V, d = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.head_dim
    specs: list[tuple[str, tuple[int, ...]]] = [("model.embed_tokens.weight", (V, H))]
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        specs += [
            (p + "input_layernorm.weight", (H,)),
            (p + "self_attn.q_proj.weight", (cfg.q_dim, H)),
            (p + "self_attn.k_proj.weight", (cfg.kv_dim, H)),
            (p + "self_attn.v_proj.weight", (cfg.kv_dim, H)),
            (p + "self_attn.o_proj.weight", (H, cfg.q_dim)),
            (p + "self_attn.q_norm.weight", (d,)),
            (p + "self_attn.k_norm.weight", (d,)),
            (p + "post_attention_layernorm.weight", (H,)),
            (p + "mlp.gate_proj.weight", (I, H)),
            (p + "mlp.up_proj.weight", (I, H)),
            (p + "mlp.down_proj.weight", (H, I)),
        ]
    specs.append(("model.norm.weight", (H,)))
    if not cfg.tie_word_embeddings:
        specs.append(("lm_head.weight", (V, H)))
    return specs


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m soc_amd.build` (HIP path unavailable)")
    L = C.CDLL(str(LIB_PATH))
    P, I32, I64, U64, F32 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64, C.c_float
    sigs = {
        "soc_last_error": (C.c_char_p, []),
        "soc_ctx_create": (C.c_int, [C.c_int, C.POINTER(P)]),
        "soc_ctx_destroy": (C.c_int, [P]),
        "soc_ctx_synchronize": (C.c_int, [P]),
        "soc_ctx_timer_start": (C.c_int, [P]),
        "soc_ctx_timer_stop": (C.c_int, [P, C.POINTER(F32)]),
        "soc_buffer_alloc": (C.c_int, [P, C.c_size_t, C.POINTER(P)]),
        "soc_buffer_free": (C.c_int, [P, P]),
        "soc_buffer_write": (C.c_int, [P, P, P, C.c_size_t]),
        "soc_buffer_read": (C.c_int, [P, P, P, C.c_size_t]),
        "soc_model_create": (C.c_int, [P, C.POINTER(QwenConfigC), C.POINTER(P)]),
        "soc_model_destroy": (C.c_int, [P]),
        "soc_model_load_tensor": (C.c_int, [P, C.c_char_p, P, I64]),
        "soc_model_synthesize": (C.c_int, [P, U64, F32]),
        "soc_model_finalize": (C.c_int, [P]),
        "soc_model_weight_bytes": (C.c_int, [P, C.POINTER(I64)]),
        "soc_model_decode_path": (C.c_int, [P, C.POINTER(I32)]),
        "soc_kv_create": (C.c_int, [P, I32, I32, C.POINTER(P)]),
        "soc_kv_destroy": (C.c_int, [P]),
        "soc_kv_length": (C.c_int, [P, I32, C.POINTER(I32)]),
        "soc_kv_reset": (C.c_int, [P, I32]),
        "soc_kv_write": (C.c_int, [P, I32, I32, I32, P, P]),
        "soc_kv_fill_synthetic": (C.c_int, [P, I32, I32, U64]),
        "soc_kv_read": (C.c_int, [P, I32, I32, P, P]),
        "soc_prefill": (C.c_int, [P, P, I32, P, I32, I32, I32, P, C.POINTER(I32)]),
        "soc_decode": (C.c_int, [P, P, I32, I32, P, C.POINTER(I32)]),
        "soc_decode_steps": (C.c_int, [P, P, I32, I32, I32, P]),
        "soc_decode_steps_noalloc": (C.c_int, [P, P, I32, I32, I32, P]),
        "soc_sample_topk": (C.c_int, [P, P, I32, I32, C.c_float, P, P, P]),
        "soc_quantize_group": (C.c_int, [P, I64, I64, I32, P, P]),
        "soc_model_quantize": (C.c_int, [P, I32]),
        "soc_bundle_open": (C.c_int, [C.c_char_p, C.POINTER(P)]),
        "soc_bundle_close": (C.c_int, [P]),
        "soc_bundle_config": (C.c_int, [P, C.POINTER(QwenConfigC)]),
        "soc_bundle_tensor_f16": (C.c_int, [P, C.c_char_p, P, I64]),
        "soc_model_load_bundle": (C.c_int, [P, C.c_char_p, C.POINTER(P)]),
        "soc_tokenizer_load": (C.c_int, [C.c_char_p, C.POINTER(P)]),
        "soc_tokenizer_load_bundle": (C.c_int, [C.c_char_p, C.POINTER(P)]),
        "soc_tokenizer_destroy": (C.c_int, [P]),
        "soc_tokenizer_encode": (C.c_int, [P, C.c_char_p, I64, P, I64, C.POINTER(I64)]),
        "soc_tokenizer_decode": (C.c_int, [P, P, I64, P, I64, C.POINTER(I64)]),
        "soc_tokenizer_token_to_id": (C.c_int, [P, C.c_char_p, I64, C.POINTER(I32)]),
        "soc_tokenizer_chat_prompt": (C.c_int, [P, P, P, I32, C.c_int, C.c_int, C.c_char_p, P, I64, C.POINTER(I64)]),
        "soc_kv_create_dims": (C.c_int, [P, I32, I32, I32, I32, I32, P]),
        "soc_kv_append": (C.c_int, [P, I32, I32, I32, I32, P, P, I32]),
        "soc_kv_set_length": (C.c_int, [P, I32, I32]),
        "soc_kv_layer_planes": (C.c_int, [P, I32, I32, P, P]),
        "soc_decode_batch": (C.c_int, [P, P, I32, P, P, P, P]),
        "soc_decode_batch_steps": (C.c_int, [P, P, I32, P, P, I32, P]),
        "soc_gemv_f16": (C.c_int, [P, P, P, P, I32, I32]),
        "soc_gemm_f16": (C.c_int, [P, P, P, P, I32, I32, I32]),
        "soc_attention_prefill": (C.c_int, [P, P, P, P, P, I32, I32, I32, I32, I32, I32]),
        "soc_attention_decode": (C.c_int, [P, P, P, P, P, I32, I32, I32, I32, I32]),
        "soc_forward": (C.c_int, [P, P, I32, P, I32, I32, P, I32, P, C.POINTER(I32)]),
        "soc_model_load_tensor_device": (C.c_int, [P, C.c_char_p, P, I32, I64]),
        "soc_model_tensor": (C.c_int, [P, C.c_char_p, C.POINTER(P), C.POINTER(I64)]),
        "soc_buffer_write_async": (C.c_int, [P, P, P, C.c_size_t]),
        "soc_op_matmul": (C.c_int, [P, P, P, P, P, P, I32, I32, I32, I32, I32]),
        "soc_op_rmsnorm": (C.c_int, [P, P, P, P, I32, I32, F32]),
        "soc_op_rope": (C.c_int, [P, P, P, I32, I32, I32, I32, I32, C.c_double]),
        "soc_op_softmax": (C.c_int, [P, P, P, I32, I32]),
        "soc_op_embedding": (C.c_int, [P, P, P, I32, P, I32, I32, I32]),
        "soc_op_mul": (C.c_int, [P, P, P, P, I32, I32]),
        "soc_qmm": (C.c_int, [P, P, P, I32, P, P, I32, I32, I32]),
        "soc_dequant": (C.c_int, [P, P, I32, P, P, I32, I32]),
        "soc_synth_normal_f16": (C.c_int, [U64, C.c_char_p, F32, I64, I64, P]),
        "soc_synth_uniform_f16": (C.c_int, [U64, C.c_char_p, F32, F32, I64, I64, P]),
        "soc_synth_tokens": (C.c_int, [U64, C.c_char_p, I32, I64, P]),
        "soc_synth_int_uniform": (C.c_int, [U64, C.c_char_p, I32, I32, I64, P]),
        "soc_synth_codes": (C.c_int, [U64, C.c_char_p, I32, I64, P]),
        "soc_f64_to_f16_rne": (C.c_uint16, [C.c_double]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != SOC_OK:
        raise SocError(rc, lib().soc_last_error().decode(errors="replace"))


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---- seeded generator --------------------------------------------------------------------------------------
def synth_normal_f16(seed: int, name: str, sigma: float, n: int, offset: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    check(lib().soc_synth_normal_f16(seed, name.encode(), sigma, offset, n, _ptr(out)))
    return out


def synth_uniform_f16(seed: int, name: str, lo: float, hi: float, n: int, offset: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    check(lib().soc_synth_uniform_f16(seed, name.encode(), lo, hi, offset, n, _ptr(out)))
    return out


def synth_tokens(seed: int, name: str, vocab: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    check(lib().soc_synth_tokens(seed, name.encode(), vocab, n, _ptr(out)))
    return out


def synth_int_uniform(seed: int, name: str, lo: int, hi: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    check(lib().soc_synth_int_uniform(seed, name.encode(), lo, hi, n, _ptr(out)))
    return out


def synth_codes(seed: int, name: str, bits: int, n_codes: int) -> np.ndarray:
    out = np.empty(n_codes if bits == 8 else n_codes // 2, dtype=np.uint8)
    check(lib().soc_synth_codes(seed, name.encode(), bits, n_codes, _ptr(out)))
    return out


def synth_weights(cfg: QwenConfig, seed: int, sigma: float = 0.02) -> dict[str, np.ndarray]:
    """Host copies of the weights soc_model_synthesize uploads (norm gains 1.0, everything else N(0, sigma))."""
    out = {}
    for name, shape in tensor_specs(cfg):
        n = int(np.prod(shape))
        if name.endswith("norm.weight"):
            out[name] = np.full(shape, 0x3C00, dtype=np.uint16)
        else:
            out[name] = synth_normal_f16(seed, name, sigma, n).reshape(shape)
    return out


# ---- objects -------------------------------------------------------------------------------------------------
class Context:
    """HIP device context (one stream)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib().soc_ctx_create(device, C.byref(h)))
        self.h = h

    def close(self) -> None:
        if self.h:
            lib().soc_ctx_destroy(self.h)
            self.h = None

    def synchronize(self) -> None:
        check(lib().soc_ctx_synchronize(self.h))

    def timer_start(self) -> None:
        check(lib().soc_ctx_timer_start(self.h))

    def timer_stop(self) -> float:
        ms = C.c_float()
        check(lib().soc_ctx_timer_stop(self.h, C.byref(ms)))
        return ms.value

    # device buffers
    def alloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        check(lib().soc_buffer_alloc(self.h, nbytes, C.byref(p)))
        return p.value

    def free(self, p: int) -> None:
        check(lib().soc_buffer_free(self.h, p))

    def upload(self, arr: np.ndarray) -> int:
        arr = np.ascontiguousarray(arr)
        p = self.alloc(arr.nbytes)
        check(lib().soc_buffer_write(self.h, p, _ptr(arr), arr.nbytes))
        return p

    def write(self, p: int, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        check(lib().soc_buffer_write(self.h, p, _ptr(arr), arr.nbytes))

    def download(self, p: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        check(lib().soc_buffer_read(self.h, _ptr(out), p, out.nbytes))
        return out

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Model:
    """Device-resident Qwen3 weights (fp16), loaded by Hugging Face tensor name."""

    def __init__(self, ctx: Context, cfg: QwenConfig):
        self.ctx, self.cfg = ctx, cfg
        h = C.c_void_p()
        c = cfg.to_c()
        check(lib().soc_model_create(ctx.h, C.byref(c), C.byref(h)))
        self.h = h

    @classmethod
    def wrap(cls, ctx: Context, cfg: QwenConfig, handle) -> "Model":
        """A Model around a soc_model the library created (soc_model_load_bundle)."""
        m = cls.__new__(cls)
        m.ctx, m.cfg, m.h = ctx, cfg, handle
        return m

    def load(self, weights: dict[str, np.ndarray]) -> "Model":
        for name, arr in weights.items():
            a = np.ascontiguousarray(arr).view(np.uint16)
            check(lib().soc_model_load_tensor(self.h, name.encode(), _ptr(a), a.size))
        check(lib().soc_model_finalize(self.h))
        return self

    def synthesize(self, seed: int, sigma: float = 0.02) -> "Model":
        check(lib().soc_model_synthesize(self.h, seed, sigma))
        check(lib().soc_model_finalize(self.h))
        return self

    def quantize(self, bits: int) -> "Model":
        """Group-64 int8 / int4 projections (soc_model_quantize)."""
        check(lib().soc_model_quantize(self.h, bits))
        return self

    def weight_bytes(self) -> int:
        v = C.c_int64()
        check(lib().soc_model_weight_bytes(self.h, C.byref(v)))
        return v.value

    def decode_path(self) -> str:
        """"xcd" (one k_decode_xcd launch per token, each layer split over the 8 XCDs), "persistent" (one
        k_decode_persistent launch per token) or "graph" (per-operator kernels)."""
        v = C.c_int32()
        check(lib().soc_model_decode_path(self.h, C.byref(v)))
        return {2: "xcd", 1: "persistent"}.get(v.value, "graph")

    def close(self) -> None:
        if self.h:
            lib().soc_model_destroy(self.h)
            self.h = None


class KVCache:
    """fp16 KV cache with `slots` independent sequences of `capacity` positions."""

    def __init__(self, model: Model, slots: int, capacity: int):
        self.model, self.slots, self.capacity = model, slots, capacity
        h = C.c_void_p()
        check(lib().soc_kv_create(model.h, slots, capacity, C.byref(h)))
        self.h = h

    def length(self, slot: int = 0) -> int:
        v = C.c_int32()
        check(lib().soc_kv_length(self.h, slot, C.byref(v)))
        return v.value

    def reset(self, slot: int = 0) -> None:
        check(lib().soc_kv_reset(self.h, slot))

    def write(self, slot: int, layer: int, pos: int, key: np.ndarray, value: np.ndarray) -> None:
        k = np.ascontiguousarray(key, dtype=np.float32)
        v = np.ascontiguousarray(value, dtype=np.float32)
        check(lib().soc_kv_write(self.h, slot, layer, pos, _ptr(k), _ptr(v)))

    def fill_synthetic(self, slot: int, length: int, seed: int) -> None:
        check(lib().soc_kv_fill_synthetic(self.h, slot, length, seed))

    def read(self, slot: int, layer: int) -> tuple[np.ndarray, np.ndarray]:
        cfg = self.model.cfg
        n = self.length(slot)
        k = np.empty((cfg.num_key_value_heads, n, cfg.head_dim), dtype=np.float16)
        v = np.empty_like(k)
        check(lib().soc_kv_read(self.h, slot, layer, _ptr(k), _ptr(v)))
        return k, v

    def close(self) -> None:
        if self.h:
            lib().soc_kv_destroy(self.h)
            self.h = None


def prefill(model: Model, kv: KVCache, slot: int, ids, position_offset: int | None = None,
            logit_rows: int = 1) -> tuple[np.ndarray | None, int]:
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    if position_offset is None:
        position_offset = kv.length(slot)
    logits = np.empty((logit_rows, model.cfg.vocab_size), dtype=np.float32) if logit_rows > 0 else None
    tok = C.c_int32()
    check(lib().soc_prefill(model.h, kv.h, slot, _ptr(ids), ids.size, position_offset, logit_rows,
                            _ptr(logits) if logits is not None else None, C.byref(tok)))
    return logits, tok.value


def decode(model: Model, kv: KVCache, slot: int, last_token: int, want_logits: bool = True):
    logits = np.empty(model.cfg.vocab_size, dtype=np.float32) if want_logits else None
    tok = C.c_int32()
    check(lib().soc_decode(model.h, kv.h, slot, int(last_token), _ptr(logits) if logits is not None else None,
                           C.byref(tok)))
    return logits, tok.value


def decode_steps(model: Model, kv: KVCache, slot: int, last_token: int, steps: int) -> np.ndarray:
    out = np.empty(steps, dtype=np.int32)
    check(lib().soc_decode_steps(model.h, kv.h, slot, int(last_token), steps, _ptr(out)))
    return out


def decode_steps_noalloc(model: Model, kv: KVCache, slot: int, last_token: int, steps: int) -> np.ndarray:
    """decode_steps through soc_decode_steps_noalloc (device buffers from the library's static scratch array)."""
    out = np.empty(steps, dtype=np.int32)
    check(lib().soc_decode_steps_noalloc(model.h, kv.h, slot, int(last_token), steps, _ptr(out)))
    return out


class Bundle:
    """A model bundle on disk (manifest.json + raw tensor files), opened and validated without a GPU."""

    def __init__(self, manifest_path):
        self.h = None
        h = C.c_void_p()
        check(lib().soc_bundle_open(str(manifest_path).encode(), C.byref(h)))
        self.h = h

    def close(self) -> None:
        if self.h:
            lib().soc_bundle_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def config(self) -> QwenConfig:
        c = QwenConfigC()
        check(lib().soc_bundle_config(self.h, C.byref(c)))
        return QwenConfig(c.vocab_size, c.hidden_size, c.num_hidden_layers, c.num_attention_heads,
                          c.num_key_value_heads, c.intermediate_size, c.head_dim, c.max_position_embeddings,
                          c.rope_theta, float(c.rms_norm_eps), bool(c.tie_word_embeddings))

    def tensor_f16(self, name: str, shape) -> np.ndarray:
        out = np.empty(shape, dtype=np.uint16)
        check(lib().soc_bundle_tensor_f16(self.h, name.encode(), _ptr(out), out.size))
        return out


def load_bundle(ctx: Context, manifest_path) -> "Model":
    """A finalized model from a bundle (soc_model_load_bundle)."""
    h = C.c_void_p()
    check(lib().soc_model_load_bundle(ctx.h, str(manifest_path).encode(), C.byref(h)))
    b = Bundle(manifest_path)
    try:
        cfg = b.config()
    finally:
        b.close()
    return Model.wrap(ctx, cfg, h)


class Tokenizer:
    """The bundle's tokenizer runtime and Qwen3 chat template (soc_tokenizer_*); host only, no GPU needed.

    Tokenizer(runtime_json_path) reads one tokenizer_runtime.json; Tokenizer.from_bundle(manifest_path) reads the file
    a manifest names and validates the two together. Text is str (UTF-8) or bytes; decode returns bytes, since a
    token sequence need not end on a character boundary."""

    def __init__(self, runtime_path=None, *, _handle=None):
        self.h = None
        if _handle is None:
            h = C.c_void_p()
            check(lib().soc_tokenizer_load(str(runtime_path).encode(), C.byref(h)))
            _handle = h
        self.h = _handle

    @classmethod
    def from_bundle(cls, manifest_path) -> "Tokenizer":
        h = C.c_void_p()
        check(lib().soc_tokenizer_load_bundle(str(manifest_path).encode(), C.byref(h)))
        return cls(_handle=h)

    def close(self) -> None:
        if self.h:
            lib().soc_tokenizer_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def encode(self, text) -> list[int]:
        b = text.encode() if isinstance(text, str) else bytes(text)
        # one id per byte, plus one per BPE segment when a prefix space is added: 2 * len + 1 always suffices
        out = np.empty(2 * len(b) + 1, np.int32)
        n = C.c_int64()
        check(lib().soc_tokenizer_encode(self.h, b, len(b), _ptr(out), out.size, C.byref(n)))
        return out[: n.value].tolist()

    def decode(self, ids) -> bytes:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        n = C.c_int64()
        rc = lib().soc_tokenizer_decode(self.h, _ptr(a), a.size, None, 0, C.byref(n))
        if rc != 0 and n.value == 0:
            check(rc)
        buf = C.create_string_buffer(max(1, n.value))
        check(lib().soc_tokenizer_decode(self.h, _ptr(a), a.size, buf, n.value, C.byref(n)))
        return buf.raw[: n.value]

    def token_to_id(self, token) -> int:
        b = token.encode() if isinstance(token, str) else bytes(token)
        out = C.c_int32()
        check(lib().soc_tokenizer_token_to_id(self.h, b, len(b), C.byref(out)))
        return out.value

    def chat_prompt(self, messages, add_generation_prompt=True, enable_thinking=True, system_prompt=None) -> bytes:
        """Qwen3TemplateBuilder::BuildPrompt over [(role, content), ...]."""
        enc = [(r.encode(), c.encode()) for r, c in messages]
        roles = (C.c_char_p * max(1, len(enc)))(*[r for r, _ in enc])
        contents = (C.c_char_p * max(1, len(enc)))(*[c for _, c in enc])
        sp = system_prompt.encode() if system_prompt else None
        n = C.c_int64()
        args = (self.h, C.cast(roles, C.c_void_p), C.cast(contents, C.c_void_p), len(enc), int(add_generation_prompt),
                int(enable_thinking), sp)
        rc = lib().soc_tokenizer_chat_prompt(*args, None, 0, C.byref(n))
        if rc != 0 and n.value == 0:
            check(rc)
        buf = C.create_string_buffer(max(1, n.value))
        check(lib().soc_tokenizer_chat_prompt(*args, buf, n.value, C.byref(n)))
        return buf.raw[: n.value]


def quantize_group(w_f16: np.ndarray, bits: int) -> tuple[np.ndarray, np.ndarray]:
    """The library's group-64 packer (soc_quantize_group) on fp16 weight rows [n][k]."""
    w = np.ascontiguousarray(w_f16).view(np.uint16)
    n, k = w.shape
    codes = np.empty((n, k) if bits == 8 else (n, k // 2), np.int8 if bits == 8 else np.uint8)
    scales = np.empty((n, k // 64), np.uint16)
    check(lib().soc_quantize_group(_ptr(w), n, k, bits, _ptr(codes), _ptr(scales)))
    return codes, scales


def sample_topk(ctx: Context, row_ptr: int, vocab: int, top_k: int, temperature: float = 1.0):
    """soc_sample_topk on a device logits row: (token, candidate ids, their raw logits)."""
    k = max(1, min(int(top_k), int(vocab)))
    ids = np.empty(k, np.int32)
    vals = np.empty(k, np.float32)
    tok = C.c_int32()
    check(lib().soc_sample_topk(ctx.h, row_ptr, vocab, top_k, temperature, C.byref(tok), _ptr(ids), _ptr(vals)))
    return tok.value, ids, vals


def decode_batch(model: Model, kv: KVCache, slots, tokens, want_logits: bool = True):
    """One ragged decode step: row i feeds tokens[i] to slot slots[i] at that slot's current length.
    Returns (logits [n][V] or None, next tokens [n])."""
    slots = np.ascontiguousarray(slots, dtype=np.int32)
    tokens = np.ascontiguousarray(tokens, dtype=np.int32)
    n = int(slots.size)
    logits = np.empty((n, model.cfg.vocab_size), dtype=np.float32) if want_logits else None
    nxt = np.empty(n, dtype=np.int32)
    check(lib().soc_decode_batch(model.h, kv.h, n, _ptr(slots), _ptr(tokens),
                                 _ptr(logits) if logits is not None else None, _ptr(nxt)))
    return logits, nxt


def decode_batch_steps(model: Model, kv: KVCache, slots, tokens, steps: int) -> np.ndarray:
    """`steps` greedy ragged decode steps, tokens fed back on the device. Returns [steps][n] token ids."""
    slots = np.ascontiguousarray(slots, dtype=np.int32)
    tokens = np.ascontiguousarray(tokens, dtype=np.int32)
    n = int(slots.size)
    out = np.empty((steps, n), dtype=np.int32)
    check(lib().soc_decode_batch_steps(model.h, kv.h, n, _ptr(slots), _ptr(tokens), steps, _ptr(out)))
    return out


def gemv_f16(ctx: Context, w_dev: int, x_dev: int, y_dev: int, n: int, k: int) -> None:
    check(lib().soc_gemv_f16(ctx.h, w_dev, x_dev, y_dev, n, k))


def qmm(ctx: Context, x_dev: int, codes_dev: int, bits: int, scales_dev: int, y_dev: int, m: int, n: int,
        k: int) -> None:
    check(lib().soc_qmm(ctx.h, x_dev, codes_dev, bits, scales_dev, y_dev, m, n, k))


def dequant(ctx: Context, codes_dev: int, bits: int, scales_dev: int, w_dev: int, n: int, k: int) -> None:
    check(lib().soc_dequant(ctx.h, codes_dev, bits, scales_dev, w_dev, n, k))


def forward(model: Model, kv: "KVCache | None", slot: int, ids, position_offset: int, want_hidden: bool = False,
            logit_rows: int = 1, ids_dev: int | None = None):
    """soc_forward (QwenCausalLM::Forward{Hidden,Logits}[Cached]): kv None = the uncached forward. Token ids from the
    host array `ids`, or from device memory at ids_dev (len(ids) of them). Returns (hidden [n][H] or None,
    logits [logit_rows][V] or None, greedy token of the last row)."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    n = int(ids.size)
    hidden = np.empty((n, model.cfg.hidden_size), np.float32) if want_hidden else None
    logits = np.empty((logit_rows, model.cfg.vocab_size), np.float32) if logit_rows > 0 else None
    tok = C.c_int32()
    check(lib().soc_forward(model.h, kv.h if kv is not None else None, slot,
                            ids_dev if ids_dev is not None else _ptr(ids), n, position_offset,
                            _ptr(hidden) if hidden is not None else None, logit_rows,
                            _ptr(logits) if logits is not None else None, C.byref(tok)))
    return hidden, logits, tok.value


def gemm_f16(ctx: Context, x_dev: int, w_dev: int, y_dev: int, m: int, n: int, k: int) -> None:
    """soc_gemm_f16: y[m][n] = x[m][k] . w[n][k]^T (fp16 operands, fp32 out), the prefill projection GEMM."""
    check(lib().soc_gemm_f16(ctx.h, x_dev, w_dev, y_dev, m, n, k))


def attention_prefill(ctx: Context, q_dev: int, k_dev: int, v_dev: int, out_dev: int, rows: int, pos_base: int,
                      nq: int, nkv: int, cap: int) -> None:
    check(lib().soc_attention_prefill(ctx.h, q_dev, k_dev, v_dev, out_dev, rows, pos_base, nq, nkv, 128, cap))


def attention_decode(ctx: Context, q_dev: int, k_dev: int, v_dev: int, out_dev: int, kv_len: int, nq: int, nkv: int,
                     cap: int) -> None:
    check(lib().soc_attention_decode(ctx.h, q_dev, k_dev, v_dev, out_dev, kv_len, nq, nkv, 128, cap))
