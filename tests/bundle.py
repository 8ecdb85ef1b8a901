"""Writes model bundles in the reference's export format for tests (the manifest + raw tensor files that
Mac/cpu/test/test_model_loader.cpp:17-105 writes for its loader tests): manifest.json with format
"soc.cpp.llm_export", format_version 2, the Hugging Face config, and one little-endian file per tensor."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bfloat16 bits, round to nearest even (finite inputs)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def encode(values: np.ndarray, dtype: str) -> bytes:
    """Raw file contents of `values` (fp32 numbers, or fp16 bits when values.dtype is uint16) stored as dtype."""
    v = np.asarray(values)
    if v.dtype == np.uint16:  # fp16 bits
        f = v.view(np.float16).astype(np.float32)
    else:
        f = v.astype(np.float32)
    if dtype == "float32":
        return f.astype("<f4").tobytes()
    if dtype == "float16":
        return (v if v.dtype == np.uint16 else f.astype(np.float16).view(np.uint16)).astype("<u2").tobytes()
    if dtype == "bfloat16":
        return f32_to_bf16_bits(f).astype("<u2").tobytes()
    if dtype == "int32":
        return v.astype("<i4").tobytes()
    raise ValueError(dtype)


def config_dict(cfg, torch_dtype: str = "float16", **extra) -> dict:
    d = {"model_type": "qwen3", "hidden_size": cfg.hidden_size, "intermediate_size": cfg.intermediate_size,
         "num_hidden_layers": cfg.num_hidden_layers, "num_attention_heads": cfg.num_attention_heads,
         "num_key_value_heads": cfg.num_key_value_heads, "head_dim": cfg.head_dim,
         "rms_norm_eps": cfg.rms_norm_eps, "rope_theta": cfg.rope_theta,
         "tie_word_embeddings": bool(cfg.tie_word_embeddings), "torch_dtype": torch_dtype,
         "vocab_size": cfg.vocab_size, "max_position_embeddings": cfg.max_position_embeddings}
    d.update(extra)
    return d


def write_bundle(root: Path, config: dict, tensors: dict[str, tuple[np.ndarray, str]], *, export_dtype="float16",
                 manifest_overrides: dict | None = None, byte_size_delta: dict[str, int] | None = None,
                 truncate: dict[str, int] | None = None, drop: tuple[str, ...] = (),
                 tokenizer_runtime: dict | None = None, generation_config: dict | None = None) -> Path:
    """tensors: name -> (values with their shape, file dtype); manifest_overrides / drop replace or remove top-level
    manifest keys; tokenizer_runtime, when given, is written as tokenizer/tokenizer_runtime.json (the file the
    manifest names). Returns the manifest path."""
    root = Path(root)
    (root / "weights").mkdir(parents=True, exist_ok=True)
    records = []
    for i, (name, (values, dtype)) in enumerate(tensors.items()):
        data = encode(values, dtype)
        if truncate and name in truncate:
            data = data[:truncate[name]]
        rel = f"weights/t{i:04d}.bin"
        (root / rel).write_bytes(data)
        size = int(np.prod(np.asarray(values).shape)) * {"float32": 4, "int32": 4}.get(dtype, 2)
        records.append({"name": name, "file": rel, "dtype": dtype, "shape": list(np.asarray(values).shape),
                        "byte_size": size + (byte_size_delta or {}).get(name, 0),
                        "source_shard": "model-00001-of-00001.safetensors"})
    manifest = {"format": "soc.cpp.llm_export", "format_version": 2, "model_id": "test/qwen3",
                "source_dir": str(root), "export_dtype": export_dtype,
                "tokenizer_runtime_file": "tokenizer/tokenizer_runtime.json", "config": config,
                "generation_config": generation_config or {}, "tensors": records}
    manifest.update(manifest_overrides or {})
    for key in drop:
        del manifest[key]
    if tokenizer_runtime is not None:
        (root / "tokenizer").mkdir(exist_ok=True)
        (root / "tokenizer" / "tokenizer_runtime.json").write_text(
            json.dumps(tokenizer_runtime, indent=1, ensure_ascii=False), encoding="utf-8")
    path = root / "manifest.json"
    path.write_text(json.dumps(manifest, indent=1))
    return path
