"""Test infrastructure, not product code: a CPU restatement of the reference's model-export
writer, used by tests to make export directories for the product's loader
(``mla_export_read`` / ``mla_model_load`` / ``mla_engine_load``) to read back.

Restated from the reference (file:line):
  * ``save`` for ``export_model`` (src/train/checkpoint.cpp:108-179, 182-185): weights.bin,
    tokenizer.json (the tokenizer file's bytes), config.json, manifest.json, COMPLETE;
  * ``TensorWriter::add`` (src/train/checkpoint.cpp:56-83): one entry per parameter,
    contiguous offsets, CRC32 of the stored bytes, f16 = IEEE round-to-nearest-even with
    a +-65504 range check, f32 as is; non-finite tensors are refused;
  * ``ModelConfig::json`` / ``hash`` (src/model/config.cpp:49-73): the architecture
    object and the SHA-256 of its compact dump;
  * ``Json::dump`` and ``quote`` (src/core/json.cpp:222-293): sorted keys, numbers as
    doubles with 17 significant digits, the reference's string escapes; ``write_json``
    appends a newline (src/core/json.cpp:363);
  * parameter names and roles (src/model/model.cpp:9-19, 26-63).

Pinned in tests/test_export.py against the reference's own records
(tests/golden/export_*.json, from docs/verification/{pretrain-cpu,full-model-pilot}):
the config hash, the tokenizer hash and every weights.bin entry's name, role, shape,
dtype, offset and size.  SHA-256 and CRC-32 come from Python's hashlib and zlib (the
same FIPS 180-4 and IEEE 802.3 reflected-polynomial definitions the reference uses).
"""
from __future__ import annotations

import hashlib
import math
import os
import zlib

import numpy as np

LAYER_TENSORS = [("attn.norm", "norm_scale"), ("attn.w_dq", "hidden_matrix"),
                 ("attn.q_norm", "norm_scale"), ("attn.w_uq", "hidden_matrix"),
                 ("attn.w_dkv", "hidden_matrix"), ("attn.kv_norm", "norm_scale"),
                 ("attn.w_uk", "hidden_matrix"), ("attn.w_uv", "hidden_matrix"),
                 ("attn.w_o", "hidden_matrix"), ("ffn.norm", "norm_scale"),
                 ("ffn.w_gate", "hidden_matrix"), ("ffn.w_up", "hidden_matrix"),
                 ("ffn.w_down", "hidden_matrix")]


def quote(s: str) -> str:
    """json.cpp:222-254: escapes for quote, backslash, \\n, \\r, \\t and other bytes
    below 32 (\\u00xx); every other byte is copied."""
    out = ['"']
    for ch in s:
        c = ord(ch)
        if ch == '"':
            out.append('\\"')
        elif ch == "\\":
            out.append("\\\\")
        elif ch == "\n":
            out.append("\\n")
        elif ch == "\r":
            out.append("\\r")
        elif ch == "\t":
            out.append("\\t")
        elif c < 32:
            out.append("\\u00%02x" % c)
        else:
            out.append(ch)
    out.append('"')
    return "".join(out)


def dump(v) -> str:
    """Json::dump (json.cpp:263-293): every number is a double printed with 17
    significant digits (std::setprecision(17)), object keys in sorted order."""
    if v is None:
        return "null"
    if isinstance(v, bool):
        return "true" if v else "false"
    if isinstance(v, (int, float, np.integer, np.floating)):
        x = float(v)
        if not math.isfinite(x):
            raise ValueError("Nonfinite JSON number")
        return "%.17g" % x
    if isinstance(v, str):
        return quote(v)
    if isinstance(v, (list, tuple)):
        return "[" + ",".join(dump(x) for x in v) + "]"
    if isinstance(v, dict):
        return "{" + ",".join(quote(k) + ":" + dump(v[k]) for k in sorted(v)) + "}"
    raise TypeError(type(v))


def config_json(cfg: dict) -> dict:
    """ModelConfig::json (config.cpp:49-70); epsilon and theta are floats in the
    reference's struct, widened to double for the dump."""
    j = {"model_type": "mla_dense_decoder", "version": 1}
    for k in ("vocab_size", "max_sequence_length", "n_layers", "d_model", "n_heads",
              "head_dim_nope", "head_dim_rope", "head_dim_value", "q_lora_rank",
              "kv_lora_rank", "d_ff"):
        j[k] = int(cfg[k])
    j["norm_epsilon"] = float(np.float32(cfg["norm_epsilon"]))
    j["rope_theta"] = float(np.float32(cfg["rope_theta"]))
    j.update({"norm": "rmsnorm", "activation": "swiglu", "mla_latent_norms": True,
              "bias": False, "tie_word_embeddings": True})
    return j


def config_hash(cfg: dict) -> str:
    return hashlib.sha256(dump(config_json(cfg)).encode()).hexdigest()


def tensor_list(cfg: dict):
    """(name, role, rows, cols) in registry order (model.cpp:26-63)."""
    d, q, kv, H = cfg["d_model"], cfg["q_lora_rank"], cfg["kv_lora_rank"], cfg["n_heads"]
    nope, rope, dv, ff = (cfg["head_dim_nope"], cfg["head_dim_rope"], cfg["head_dim_value"],
                          cfg["d_ff"])
    shapes = [(1, d), (d, q), (1, q), (q, H * (nope + rope)), (d, kv + rope), (1, kv),
              (kv, H * nope), (kv, H * dv), (H * dv, d), (1, d), (d, ff), (d, ff), (ff, d)]
    out = [("token_embedding", "token_embedding", cfg["vocab_size"], d),
           ("final_norm", "norm_scale", 1, d)]
    for layer in range(cfg["n_layers"]):
        for (name, role), (r, c) in zip(LAYER_TENSORS, shapes):
            out.append((f"layers.{layer}.{name}", role, r, c))
    return out


def tensor_bytes(values: np.ndarray, dtype: str) -> bytes:
    """TensorWriter::add's payload (checkpoint.cpp:56-72)."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    if not np.isfinite(values).all():
        raise ValueError("Cannot serialize nonfinite tensor")
    if dtype == "f16":
        if (np.abs(values) > 65504).any():
            raise ValueError("Tensor exceeds FP16 range")
        return values.astype("<f2").tobytes()
    if dtype == "f32":
        return values.astype("<f4").tobytes()
    raise ValueError("Export dtype must be f32 or f16")


def write_export(path: str, cfg: dict, params: np.ndarray, tokenizer_bytes: bytes,
                 dtype: str = "f16") -> dict:
    """save() for a model export (checkpoint.cpp:108-179 with no optimizer): returns the
    manifest object it wrote.  The directory must not exist yet."""
    os.makedirs(path)
    params = np.ascontiguousarray(params, dtype=np.float32).ravel()
    tensors, blobs, offset, at = [], [], 0, 0
    for name, role, r, c in tensor_list(cfg):
        raw = tensor_bytes(params[at:at + r * c], dtype)
        at += r * c
        tensors.append({"name": name, "role": role, "dtype": dtype, "shape": [r, c],
                        "file": "weights.bin", "offset": offset, "nbytes": len(raw),
                        "crc32": zlib.crc32(raw) & 0xFFFFFFFF})
        offset += len(raw)
        blobs.append(raw)
    if at != params.size:
        raise ValueError("parameter count mismatch")
    weights = b"".join(blobs)
    with open(os.path.join(path, "weights.bin"), "wb") as f:
        f.write(weights)
    with open(os.path.join(path, "tokenizer.json"), "wb") as f:
        f.write(tokenizer_bytes)
    with open(os.path.join(path, "config.json"), "w") as f:
        f.write(dump(config_json(cfg)) + "\n")
    count = sum(r * c for _, _, r, c in tensor_list(cfg))
    manifest = {"format": "mini-mla-model", "version": 1,
                "model_config_sha256": config_hash(cfg),
                "tokenizer_sha256": hashlib.sha256(tokenizer_bytes).hexdigest(),
                "parameter_count": count, "dtype": dtype, "chat_template": "mini-mla-chat-v1",
                "step": 0, "tensors": tensors,
                "sha256": {"weights.bin": hashlib.sha256(weights).hexdigest()}}
    write_manifest(path, manifest)
    return manifest


def write_manifest(path: str, manifest: dict) -> None:
    """manifest.json (write_json) and COMPLETE = SHA-256 of the manifest text + newline."""
    text = dump(manifest) + "\n"
    with open(os.path.join(path, "manifest.json"), "w") as f:
        f.write(text)
    with open(os.path.join(path, "COMPLETE"), "w") as f:
        f.write(hashlib.sha256(text.encode()).hexdigest() + "\n")
