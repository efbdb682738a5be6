"""Writes the committed golden fixtures under tests/golden/ (run in the build container).

1. ``tiny_forward.npz`` -- data held by the reference's own verification record
   ``docs/verification/attention-sync/oracle/{debug.json,tensors.bin}``: the
   tiny-test config, the 28 fp32 weight tensors in registry order, the input ids
   and the engine's logits [9 x 264] (PyTorch agreed to 2.15e-6,
   ``docs/verification/attention-sync/flash-oracle-report.json``).  Only the
   weights and logits are kept (gradients and optimizer state are dropped).
2. ``rng_vectors.json`` -- known answers of the reference's own Rng
   (``include/mini_mla/rng.hpp``) from ``oracle/_ref/rng_ref``, which
   ``oracle/Makefile`` compiles from the reference header.
3. ``export_tiny.json`` / ``export_mla36m.json`` -- the model-export contract of the
   reference's own verification records (``docs/verification/pretrain-cpu`` and
   ``docs/verification/full-model-pilot``: tiny-test and mla36m checkpoints): the
   architecture (``config/tiny-test.json``, ``config/mla36m-v1.json``), the manifest's
   ``model_config_sha256``, ``tokenizer_sha256`` and ``parameter_count``, and every
   ``weights.bin`` tensor entry (name, role, shape, dtype, offset, nbytes; the CRCs
   belong to trained weights that are not in the repository and are dropped).
   ``tokenizer_tiny.json`` / ``tokenizer_pilot.json`` are the reference's
   ``examples/tokenizer.json`` and ``examples/pilot-tokenizer.json``, byte for byte
   (their SHA-256 is the manifests' ``tokenizer_sha256``).

Usage: python tests/golden/make_fixtures.py [REFERENCE_ROOT]
"""
from __future__ import annotations

import json
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))

ORDER = ["attn.norm", "attn.w_dq", "attn.q_norm", "attn.w_uq", "attn.w_dkv", "attn.kv_norm",
         "attn.w_uk", "attn.w_uv", "attn.w_o", "ffn.norm", "ffn.w_gate", "ffn.w_up",
         "ffn.w_down"]


def tiny_forward(ref: str) -> None:
    base = os.path.join(ref, "docs", "verification", "attention-sync", "oracle")
    debug = json.load(open(os.path.join(base, "debug.json")))
    raw = open(os.path.join(base, "tensors.bin"), "rb").read()
    tensors = {e["name"]: np.frombuffer(raw[e["offset"]:e["offset"] + e["nbytes"]],
                                        dtype="<f4").reshape(e["shape"])
               for e in debug["tensors"]}
    cfg = debug["config"]
    names = ["token_embedding", "final_norm"] + [
        f"layers.{l}.{n}" for l in range(cfg["n_layers"]) for n in ORDER]
    params = np.concatenate([tensors[n + ".weight"].reshape(-1) for n in names])
    assert params.size == debug["parameter_count"], (params.size, debug["parameter_count"])
    tokens = np.array([int(x) for x in debug["input"].split(",")], dtype=np.uint16)
    logits = tensors["logits"].astype(np.float32)
    keys = ["vocab_size", "max_sequence_length", "n_layers", "d_model", "n_heads",
            "head_dim_nope", "head_dim_rope", "head_dim_value", "q_lora_rank", "kv_lora_rank",
            "d_ff", "norm_epsilon", "rope_theta"]
    np.savez_compressed(os.path.join(HERE, "tiny_forward.npz"), params=params, tokens=tokens,
                        logits=logits,
                        config=np.array(json.dumps({k: cfg[k] for k in keys})),
                        parameter_count=np.array(debug["parameter_count"]))
    print("tiny_forward.npz:", params.size, "params,", logits.shape, "logits")


def rng_vectors() -> None:
    exe = os.path.join(REPO, "oracle", "_ref", "rng_ref")
    if not os.path.exists(exe):
        raise SystemExit("oracle/_ref/rng_ref missing: run make -C oracle first")
    out = {}
    for kind, seed, count, bound in [("next", 0, 64, 0), ("next", 42, 64, 0),
                                     ("uniform", 7, 256, 0), ("normal", 0, 1024, 0),
                                     ("normal", 42, 1024, 0), ("normal", 91, 256, 0),
                                     ("bounded", 0, 256, 16384), ("bounded", 3, 256, 3969),
                                     ("bounded", 5, 64, 1), ("bounded", 9, 64, (1 << 63) + 5)]:
        vals = subprocess.run([exe, kind, str(seed), str(count), str(bound)], check=True,
                              capture_output=True, text=True).stdout.split()
        out[f"{kind}/{seed}/{bound}"] = vals
    json.dump(out, open(os.path.join(HERE, "rng_vectors.json"), "w"), indent=0)
    print("rng_vectors.json:", len(out), "series")


def export_fixtures(ref: str) -> None:
    for name, record, config, tok in [
            ("tiny", "pretrain-cpu", "tiny-test.json", "tokenizer.json"),
            ("mla36m", "full-model-pilot", "mla36m-v1.json", "pilot-tokenizer.json")]:
        m = json.load(open(os.path.join(ref, "docs", "verification", record, "manifest.json")))
        arch = json.load(open(os.path.join(ref, "config", config)))
        tensors = [{k: e[k] for k in ("name", "role", "shape", "dtype", "offset", "nbytes")}
                   for e in m["tensors"] if e["file"] == "weights.bin"]
        out = {"source": f"docs/verification/{record}/manifest.json, config/{config}",
               "config": arch, "model_config_sha256": m["model_config_sha256"],
               "tokenizer_sha256": m["tokenizer_sha256"],
               "parameter_count": m["parameter_count"], "weights": tensors}
        json.dump(out, open(os.path.join(HERE, f"export_{name}.json"), "w"), indent=0)
        raw = open(os.path.join(ref, "examples", tok), "rb").read()
        dst = "tokenizer_tiny.json" if name == "tiny" else "tokenizer_pilot.json"
        open(os.path.join(HERE, dst), "wb").write(raw)
        print(f"export_{name}.json: {len(tensors)} tensors; {dst}: {len(raw)} bytes")


if __name__ == "__main__":
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    what = sys.argv[2:] or ["tiny_forward", "rng_vectors", "export_fixtures"]
    for fn in what:
        globals()[fn](ref)
