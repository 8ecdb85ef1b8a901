"""ctypes binding of the CPU oracle. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may import this module. It wraps:
  * oracle/liboracle.so   - this project's restatement of the reference CPU arithmetic (soc_oracle.cpp)
  * oracle/_ref/libsocref.so - the reference's own CPU sources compiled from /root/reference with ref_driver.cpp
    (present only where `make -C oracle ref` could run; absent on machines without the reference checkout)

Both expose the same operations; `Oracle(kind="port")` and `Oracle(kind="reference")` select the library.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
PORT_LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libsocref.so"

P, I32, I64, F32, F64 = C.c_void_p, C.c_int32, C.c_int64, C.c_float, C.c_double


def build(ref: bool = True) -> None:
    """Builds liboracle.so (and _ref/libsocref.so when the reference checkout exists)."""
    targets = ["oracle"] + (["ref"] if ref else [])
    subprocess.run(["make", "-s", "-C", str(HERE), *targets], check=True)


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


_port = None
_ref = None


def port_lib() -> C.CDLL:
    global _port
    if _port is None:
        if not PORT_LIB.exists():
            build(ref=False)
        L = C.CDLL(str(PORT_LIB))
        sigs = {
            "orc_f16_to_f32": (F32, [C.c_uint16]),
            "orc_f32_to_f16": (C.c_uint16, [F32]),
            "orc_f16_to_f32_array": (None, [P, P, I64]),
            "orc_linear_f16": (None, [P, I64, I64, P, I64, P]),
            "orc_linear_f32": (None, [P, I64, I64, P, I64, P]),
            "orc_rmsnorm_f16": (None, [P, I64, I64, P, F32, P]),
            "orc_rmsnorm_f32": (None, [P, I64, I64, P, F32, P]),
            "orc_rope": (None, [P, I64, I64, I64, F64, I64]),
            "orc_gqa": (C.c_int, [P, P, P, I64, I64, I64, I64, I64, I64, C.c_int, P]),
            "orc_sample": (C.c_int, [P, I64, F32, I64]),
            "orc_sample_topk": (C.c_int, [P, I64, F32, I64, P, P]),
            "orc_quantize_group": (C.c_int, [P, I64, I64, C.c_int, P, P]),
            "orc_model_set_f32": (C.c_int, [P, C.c_char_p, P, I64]),
            "orc_mlp_f16": (None, [P, I64, I64, I64, P, P, P, P]),
            "orc_model_create": (P, [I64, I64, I64, I64, I64, I64, I64, F64, F32, C.c_int]),
            "orc_model_destroy": (None, [P]),
            "orc_model_set": (C.c_int, [P, C.c_char_p, P, I64]),
            "orc_model_check": (C.c_int, [P]),
            "orc_cache_create": (P, [P, I64]),
            "orc_cache_destroy": (None, [P]),
            "orc_cache_clear": (None, [P]),
            "orc_cache_length": (I64, [P]),
            "orc_cache_write": (C.c_int, [P, I64, I64, P, P]),
            "orc_forward_logits": (C.c_int, [P, P, I64, I64, P, P]),
            "orc_forward_logits_cached": (C.c_int, [P, P, P, I64, I64, I64, P]),
            "orc_generate": (C.c_int, [P, P, I64, I64, C.c_int, I64, F32, I64, P, P]),
            "orc_qmm_group": (C.c_int, [P, I64, I64, P, C.c_int, P, I64, I64, P]),
            "orc_dequant_group": (C.c_int, [P, C.c_int, P, I64, I64, I64, P]),
            "orc_quant_int8_percol": (None, [P, I64, I64, P, P]),
            "orc_matmul_quant_int8": (None, [P, I64, I64, P, P, I64, P]),
            "orc_set_threads": (C.c_int, [C.c_int]),
        }
        for n, (r, a) in sigs.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        _port = L
    return _port


def ref_available() -> bool:
    return REF_LIB.exists()


def ref_lib() -> C.CDLL:
    global _ref
    if _ref is None:
        if not REF_LIB.exists():
            raise FileNotFoundError(f"{REF_LIB} not built (needs the reference checkout; `make -C oracle ref`)")
        L = C.CDLL(str(REF_LIB))
        sigs = {
            "ref_last_error": (C.c_char_p, []),
            "ref_f16_to_f32": (F32, [C.c_uint16]),
            "ref_f32_to_f16": (C.c_uint16, [F32]),
            "ref_f16_to_f32_array": (None, [P, P, I64]),
            "ref_f32_to_f16_array": (None, [P, P, I64]),
            "ref_linear_f16": (C.c_int, [P, I64, I64, P, I64, P]),
            "ref_rmsnorm_f16": (C.c_int, [P, I64, I64, P, F32, P]),
            "ref_rope": (C.c_int, [P, I64, I64, I64, F64, I64]),
            "ref_gqa": (C.c_int, [P, P, P, I64, I64, I64, I64, I64, I64, C.c_int, P]),
            "ref_sample": (C.c_int, [P, I64, F32, I64]),
            "ref_model_create": (P, [I64, I64, I64, I64, I64, I64, I64, F64, F32, C.c_int, P, P, C.c_int]),
            "ref_model_destroy": (None, [P]),
            "ref_cache_create": (P, [P, I64]),
            "ref_cache_destroy": (None, [P]),
            "ref_cache_write": (C.c_int, [P, I64, I64, P, P, I64, I64]),
            "ref_forward_logits": (C.c_int, [P, P, I64, I64, P]),
            "ref_forward_logits_cached": (C.c_int, [P, P, P, I64, I64, P]),
            "ref_generate": (C.c_int, [P, P, I64, I64, C.c_int, I64, F32, I64, P, P]),
            "ref_quant_matmul_int8": (C.c_int, [P, I64, I64, P, I64, P, P, P]),
        }
        for n, (r, a) in sigs.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        _ref = L
    return _ref


def set_threads(n: int) -> int:
    return port_lib().orc_set_threads(n)


# ---- ops (port) ----------------------------------------------------------------------------------------------
def f16_to_f32(codes: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.uint16)
    out = np.empty(c.shape, dtype=np.float32)
    port_lib().orc_f16_to_f32_array(_ptr(c), _ptr(out), c.size)
    return out


def f32_to_f16(x: float) -> int:
    return port_lib().orc_f32_to_f16(x)


def linear_f16(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w).view(np.uint16)
    rows, k = x.reshape(-1, x.shape[-1]).shape
    n = w.shape[0]
    y = np.empty((rows, n), dtype=np.float32)
    port_lib().orc_linear_f16(_ptr(x), rows, k, _ptr(w), n, _ptr(y))
    return y.reshape(*x.shape[:-1], n)


def linear_f32(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, k = x.reshape(-1, x.shape[-1]).shape
    n = w.shape[0]
    y = np.empty((rows, n), dtype=np.float32)
    port_lib().orc_linear_f32(_ptr(x), rows, k, _ptr(w), n, _ptr(y))
    return y.reshape(*x.shape[:-1], n)


def rmsnorm_f32(x: np.ndarray, gain: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(gain, dtype=np.float32)
    y = np.empty_like(x)
    port_lib().orc_rmsnorm_f32(_ptr(x), x.size // g.size, g.size, _ptr(g), eps, _ptr(y))
    return y


def rmsnorm_f16(x: np.ndarray, gain_f16: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(gain_f16).view(np.uint16)
    y = np.empty_like(x)
    port_lib().orc_rmsnorm_f16(_ptr(x), x.size // g.size, g.size, _ptr(g), eps, _ptr(y))
    return y


def rope(x: np.ndarray, theta: float, position_offset: int) -> np.ndarray:
    """x [seq][heads][d] -> rotated copy."""
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    s, h, d = y.shape
    port_lib().orc_rope(_ptr(y), s, h, d, theta, position_offset)
    return y


def gqa(q: np.ndarray, k: np.ndarray, v: np.ndarray, prefix: int = 0, causal: bool = True) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    T, nq, d = q.shape
    S, nkv, _ = k.shape
    out = np.empty_like(q)
    rc = port_lib().orc_gqa(_ptr(q), _ptr(k), _ptr(v), T, S, nq, nkv, d, prefix, 1 if causal else 0, _ptr(out))
    if rc != 0:
        raise ValueError("orc_gqa: invalid arguments")
    return out


def sample(row: np.ndarray, temperature: float = 1.0, top_k: int = 1) -> int:
    r = np.ascontiguousarray(row, dtype=np.float32)
    return port_lib().orc_sample(_ptr(r), r.size, temperature, top_k)


def sample_topk(row: np.ndarray, temperature: float, top_k: int) -> tuple[int, np.ndarray, np.ndarray]:
    """The reference GPU sampler's result: (token, k candidate ids in its order, their raw logits)."""
    r = np.ascontiguousarray(row, dtype=np.float32)
    k = max(1, min(int(top_k), r.size))
    ids = np.empty(k, np.int32)
    vals = np.empty(k, np.float32)
    tok = port_lib().orc_sample_topk(_ptr(r), r.size, temperature, top_k, _ptr(ids), _ptr(vals))
    return tok, ids, vals


def quantize_group(w_f16: np.ndarray, bits: int) -> tuple[np.ndarray, np.ndarray]:
    """Group-64 quantization of fp16 weight rows [N][K]: (codes int8 [N][K] or packed int4 uint8 [N][K/2],
    fp16 scale bits [N][K/64])."""
    w = np.ascontiguousarray(w_f16).view(np.uint16)
    n, k = w.shape
    codes = np.zeros((n, k) if bits == 8 else (n, k // 2), np.int8 if bits == 8 else np.uint8)
    scales = np.zeros((n, k // 64), np.uint16)
    if port_lib().orc_quantize_group(_ptr(w), n, k, bits, _ptr(codes), _ptr(scales)) != 0:
        raise ValueError("orc_quantize_group: invalid arguments")
    return codes, scales


def qmm_group(a_f16: np.ndarray, codes: np.ndarray, bits: int, scales_f16: np.ndarray, k: int, n: int,
              group: int = 64) -> np.ndarray:
    a = np.ascontiguousarray(a_f16).view(np.uint16)
    m = a.size // k
    y = np.empty((m, n), dtype=np.float32)
    rc = port_lib().orc_qmm_group(_ptr(a), m, k, _ptr(np.ascontiguousarray(codes)), bits,
                                  _ptr(np.ascontiguousarray(scales_f16).view(np.uint16)), group, n, _ptr(y))
    if rc != 0:
        raise ValueError("orc_qmm_group: invalid arguments")
    return y


def dequant_group(codes: np.ndarray, bits: int, scales_f16: np.ndarray, n: int, k: int, group: int = 64) -> np.ndarray:
    w = np.empty((n, k), dtype=np.float32)
    rc = port_lib().orc_dequant_group(_ptr(np.ascontiguousarray(codes)), bits,
                                      _ptr(np.ascontiguousarray(scales_f16).view(np.uint16)), group, n, k, _ptr(w))
    if rc != 0:
        raise ValueError("orc_dequant_group: invalid arguments")
    return w


def quant_int8_percol(rhs: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    r = np.ascontiguousarray(rhs, dtype=np.float32)
    k, n = r.shape
    codes = np.empty((n, k), dtype=np.int8)
    scales = np.empty(n, dtype=np.float32)
    port_lib().orc_quant_int8_percol(_ptr(r), k, n, _ptr(codes), _ptr(scales))
    return codes, scales


def matmul_quant_int8(a: np.ndarray, codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    m, k = a.shape
    n = codes.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    port_lib().orc_matmul_quant_int8(_ptr(a), m, k, _ptr(np.ascontiguousarray(codes)),
                                     _ptr(np.ascontiguousarray(scales, dtype=np.float32)), n, _ptr(y))
    return y


# ---- model ---------------------------------------------------------------------------------------------------
class OracleModel:
    """Qwen3 forward on the CPU. kind="port" (restatement) or "reference" (compiled reference sources)."""

    def __init__(self, cfg, weights: dict[str, np.ndarray], kind: str = "port"):
        """weights: fp16 bits (uint16 / float16) by Hugging Face name; float32 arrays are fp32 projection weights
        (dequantized group-quantized ones, port only)."""
        self.cfg, self.kind = cfg, kind
        self._keep32 = {n: np.ascontiguousarray(w) for n, w in weights.items() if np.asarray(w).dtype == np.float32}
        self._keep = {n: np.ascontiguousarray(w).view(np.uint16) for n, w in weights.items() if n not in self._keep32}
        if self._keep32 and kind != "port":
            raise ValueError("fp32 projection weights are supported by the restatement only")
        args = (cfg.vocab_size, cfg.hidden_size, cfg.num_hidden_layers, cfg.num_attention_heads,
                cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size, float(cfg.rope_theta),
                float(cfg.rms_norm_eps), 1 if cfg.tie_word_embeddings else 0)
        if kind == "port":
            L = port_lib()
            self.h = L.orc_model_create(*args)
            if not self.h:
                raise ValueError("orc_model_create: invalid config")
            for n, a in self._keep.items():
                if L.orc_model_set(self.h, n.encode(), _ptr(a), a.size) != 0:
                    raise ValueError(f"orc_model_set rejected {n}")
            for n, a in self._keep32.items():
                if L.orc_model_set_f32(self.h, n.encode(), _ptr(a), a.size) != 0:
                    raise ValueError(f"orc_model_set_f32 rejected {n}")
            if L.orc_model_check(self.h) != 0:
                raise ValueError("oracle model is missing tensors")
        elif kind == "reference":
            L = ref_lib()
            names = list(self._keep)
            cnames = (C.c_char_p * len(names))(*[n.encode() for n in names])
            ptrs = (C.c_void_p * len(names))(*[_ptr(self._keep[n]) for n in names])
            self.h = L.ref_model_create(*args, cnames, ptrs, len(names))
            if not self.h:
                raise ValueError("ref_model_create: " + L.ref_last_error().decode())
        else:
            raise ValueError(kind)

    def close(self):
        if self.h:
            (port_lib().orc_model_destroy if self.kind == "port" else ref_lib().ref_model_destroy)(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward_logits(self, ids, position_offset: int = 0) -> np.ndarray:
        """Uncached forward; logits of every row [T][V]."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty((ids.size, self.cfg.vocab_size), dtype=np.float32)
        if self.kind == "port":
            rc = port_lib().orc_forward_logits(self.h, _ptr(ids), ids.size, position_offset, _ptr(out), None)
        else:
            rc = ref_lib().ref_forward_logits(self.h, _ptr(ids), ids.size, position_offset, _ptr(out))
        if rc != 0:
            raise ValueError("forward_logits failed")
        return out

    def generate(self, prompt, max_new: int, max_seq: int | None = None, eos: int = -1,
                 temperature: float = 1.0, top_k: int = 1, want_logits: bool = False):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        max_seq = max_seq or (prompt.size + max_new + 1)
        toks = np.empty(max_new, dtype=np.int32)
        logits = np.empty((max_new, self.cfg.vocab_size), dtype=np.float32) if want_logits else None
        fn = port_lib().orc_generate if self.kind == "port" else ref_lib().ref_generate
        n = fn(self.h, _ptr(prompt), prompt.size, max_new, eos, max_seq, temperature, top_k, _ptr(toks), _ptr(logits))
        if n < 0:
            raise ValueError("generate failed")
        return (toks[:n], logits[:n] if logits is not None else None)


class RefCache:
    """TensorKVCache of the compiled reference (fp32), for cached forwards of a kind="reference" model."""

    def __init__(self, model: OracleModel, max_seq: int):
        assert model.kind == "reference"
        self.model = model
        self.h = ref_lib().ref_cache_create(model.h, max_seq)
        if not self.h:
            raise ValueError("ref_cache_create: " + ref_lib().ref_last_error().decode())

    def close(self):
        if getattr(self, "h", None):
            ref_lib().ref_cache_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def write(self, layer: int, pos: int, key: np.ndarray, value: np.ndarray) -> None:
        """TensorKVCache::Write of one position's [nkv][d] keys and values (Mac/cpu/src/kv_cache.cpp:50-78)."""
        k = np.ascontiguousarray(key, dtype=np.float32)
        v = np.ascontiguousarray(value, dtype=np.float32)
        cfg = self.model.cfg
        if ref_lib().ref_cache_write(self.h, layer, pos, _ptr(k), _ptr(v), cfg.num_key_value_heads, cfg.head_dim) != 0:
            raise ValueError("ref_cache_write: " + ref_lib().ref_last_error().decode())

    def forward(self, ids, position_offset: int) -> np.ndarray:
        """QwenCausalLM::ForwardLogitsCached: logits of every row [T][V]."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty((ids.size, self.model.cfg.vocab_size), dtype=np.float32)
        if ref_lib().ref_forward_logits_cached(self.model.h, self.h, _ptr(ids), ids.size, position_offset,
                                               _ptr(out)) != 0:
            raise ValueError("ref_forward_logits_cached: " + ref_lib().ref_last_error().decode())
        return out


class OracleCache:
    """Port-oracle KV cache (fp32) for cached forwards."""

    def __init__(self, model: OracleModel, max_seq: int):
        assert model.kind == "port"
        self.model = model
        self.h = port_lib().orc_cache_create(model.h, max_seq)

    def __del__(self):
        if getattr(self, "h", None):
            port_lib().orc_cache_destroy(self.h)
            self.h = None

    def length(self) -> int:
        return port_lib().orc_cache_length(self.h)

    def write(self, layer: int, pos: int, key: np.ndarray, value: np.ndarray) -> None:
        k = np.ascontiguousarray(key, dtype=np.float32)
        v = np.ascontiguousarray(value, dtype=np.float32)
        if port_lib().orc_cache_write(self.h, layer, pos, _ptr(k), _ptr(v)) != 0:
            raise ValueError("orc_cache_write failed")

    def forward(self, ids, position_offset: int, logit_rows: int = 1) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty((logit_rows, self.model.cfg.vocab_size), dtype=np.float32)
        rc = port_lib().orc_forward_logits_cached(self.model.h, self.h, _ptr(ids), ids.size, position_offset,
                                                  logit_rows, _ptr(out))
        if rc != 0:
            raise ValueError(f"orc_forward_logits_cached failed ({rc})")
        return out
