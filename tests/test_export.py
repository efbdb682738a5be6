"""Model exports into the device model: mla_export_read / mla_model_load / mla_engine_load,
the reference's load_checkpoint(path, training=false) (src/train/checkpoint.cpp:186-324)
over its directory format (docs/file_formats.md, "Checkpoint directory").

Pinning:
  * the writer that makes the test directories (oracle/export_format.py, a restatement
    of the reference's save()) reproduces the reference's own records
    (tests/golden/export_{tiny,mla36m}.json, from docs/verification/pretrain-cpu and
    full-model-pilot): the architecture hash, the tokenizer hash and every weights.bin
    entry (name, role, shape, dtype, offset, size);
  * the product's own SHA-256 and canonical config dump reproduce the same two
    architecture hashes (mla_config_hash); its CRC-32 and SHA-256 accept every entry and
    file the writer signs with zlib / hashlib;
  * round trips are bit-exact (f32 as stored, f16 widened exactly), and every check of
    load_checkpoint fails with the reference's code and message.
All of this is host code: these tests run on the CPU.  The GPU test loads an export into
the engine and compares its logits with the engine built from the same parameters.
"""
import hashlib
import json
import os
import struct
import zlib

import numpy as np
import pytest

from conftest import GOLDEN, MLA36M, TINY


def _golden(name):
    with open(os.path.join(GOLDEN, f"export_{name}.json")) as f:
        return json.load(f)


def _tokenizer(name):
    with open(os.path.join(GOLDEN, "tokenizer_tiny.json" if name == "tiny"
                           else "tokenizer_pilot.json"), "rb") as f:
        return f.read()


def _arch(cfg_json):
    keys = ("vocab_size", "max_sequence_length", "n_layers", "d_model", "n_heads",
            "head_dim_nope", "head_dim_rope", "head_dim_value", "q_lora_rank",
            "kv_lora_rank", "d_ff", "norm_epsilon", "rope_theta")
    return {k: cfg_json[k] for k in keys}


# ------------------------------------------------------------ the writer ----
@pytest.mark.parametrize("name", ["tiny", "mla36m"])
def test_writer_reproduces_the_reference_records(name):
    from oracle import export_format as ef
    g = _golden(name)
    cfg = _arch(g["config"])
    assert ef.config_hash(cfg) == g["model_config_sha256"]
    assert hashlib.sha256(_tokenizer(name)).hexdigest() == g["tokenizer_sha256"]
    entries, offset = [], 0
    for tname, role, r, c in ef.tensor_list(cfg):
        entries.append({"name": tname, "role": role, "shape": [r, c], "dtype": "f32",
                        "offset": offset, "nbytes": 4 * r * c})
        offset += 4 * r * c
    assert entries == g["weights"]
    assert sum(e["nbytes"] for e in entries) // 4 == g["parameter_count"]


def test_writer_dump_conventions():
    """Json::dump conventions the hashes depend on (json.cpp:222-293): 17 significant
    digits, integral doubles without a point, sorted keys, the reference's escapes."""
    from oracle import export_format as ef
    assert ef.dump(1e-5) == "1.0000000000000001e-05"
    assert ef.dump(float(np.float32(1e-5))) == "9.9999997473787516e-06"
    assert ef.dump(10000.0) == "10000" and ef.dump(264) == "264"
    assert ef.dump({"b": 1, "a": [True, None, "x"]}) == '{"a":[true,null,"x"],"b":1}'
    assert ef.dump("q\"\\\n\r\t\x01/é") == '"q\\"\\\\\\n\\r\\t\\u0001/é"'
    with pytest.raises(ValueError):
        ef.dump(float("nan"))


# --------------------------------------------------------- the product ----
@pytest.mark.parametrize("name", ["tiny", "mla36m"])
def test_product_config_hash_matches_the_reference(name):
    import cpp_inference_train_engine_amd as mla
    g = _golden(name)
    assert mla.config_hash(mla.ModelConfig.from_dict(_arch(g["config"]))) == \
        g["model_config_sha256"]


def _write(tmp_path, cfg, params, tok, dtype="f16", sub="export"):
    from oracle import export_format as ef
    path = str(tmp_path / sub)
    ef.write_export(path, cfg, params, tok, dtype)
    return path


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_round_trip_tiny(tmp_path, tiny_fixture, dtype):
    """The reference's tiny-test weights (tests/golden/tiny_forward.npz) through an export:
    f32 comes back as stored, f16 as the IEEE round-to-nearest-even halves widened."""
    import cpp_inference_train_engine_amd as mla
    params = tiny_fixture["params"]
    path = _write(tmp_path, TINY, params, _tokenizer("tiny"), dtype)
    cfg, got = mla.read_export(path)
    assert cfg.to_dict() == mla.ModelConfig.from_dict(TINY).to_dict()
    want = params if dtype == "f32" else params.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(got, want)


def test_round_trip_mla36m_f16(tmp_path):
    import cpp_inference_train_engine_amd as mla
    from cpp_inference_train_engine_amd.workloads import model_params
    params = model_params(MLA36M, seed=3)
    path = _write(tmp_path, MLA36M, params, _tokenizer("mla36m"), "f16")
    cfg, got = mla.read_export(path)
    assert cfg.d_model == 512 and got.size == 35_763_840
    np.testing.assert_array_equal(got, params.astype(np.float16).astype(np.float32))


def _resign(path, manifest=None, files=("weights.bin",)):
    """Rewrites the manifest (optionally edited) with fresh file hashes and COMPLETE, so
    only the check a test targets fails."""
    from oracle import export_format as ef
    if manifest is None:
        with open(os.path.join(path, "manifest.json")) as f:
            manifest = json.load(f)
    for name in files:
        if name in manifest["sha256"]:
            with open(os.path.join(path, name), "rb") as f:
                manifest["sha256"][name] = hashlib.sha256(f.read()).hexdigest()
    ef.write_manifest(path, manifest)


def _manifest(path):
    with open(os.path.join(path, "manifest.json")) as f:
        return json.load(f)


def test_checkpoint_format_skips_training_state(tmp_path, tiny_fixture):
    """A mini-mla-checkpoint (weights + optimizer.bin + trainer_state.json) loads for
    inference; the moments are checked (hash, CRC) and skipped (checkpoint.cpp:289-290)."""
    import cpp_inference_train_engine_amd as mla
    path = _write(tmp_path, TINY, tiny_fixture["params"], _tokenizer("tiny"), "f32")
    m = _manifest(path)
    m["format"] = "mini-mla-checkpoint"
    blobs, offset = [], 0
    for e in list(m["tensors"]):
        moment = np.full(e["shape"], 0.5, np.float32).tobytes()
        m["tensors"].append({"name": "optimizer." + e["name"] + ".first", "role": e["role"],
                             "dtype": "f32", "shape": e["shape"], "file": "optimizer.bin",
                             "offset": offset, "nbytes": len(moment),
                             "crc32": zlib.crc32(moment)})
        offset += len(moment)
        blobs.append(moment)
    with open(os.path.join(path, "optimizer.bin"), "wb") as f:
        f.write(b"".join(blobs))
    with open(os.path.join(path, "trainer_state.json"), "w") as f:
        f.write("{}\n")
    m["sha256"]["optimizer.bin"] = m["sha256"]["trainer_state.json"] = ""
    _resign(path, m, ("weights.bin", "optimizer.bin", "trainer_state.json"))
    _, got = mla.read_export(path)
    np.testing.assert_array_equal(got, tiny_fixture["params"])


def _flip(path, name, at):
    with open(os.path.join(path, name), "r+b") as f:
        f.seek(at)
        b = f.read(1)
        f.seek(at)
        f.write(bytes([b[0] ^ 0x01]))


def _corrupt(path, case):
    """Applies one defect; returns (error code, message prefix) the reference gives."""
    m = _manifest(path)
    t = m["tensors"]
    if case == "no_manifest":
        os.remove(os.path.join(path, "manifest.json"))
        return "io_error", os.path.join(path, "manifest.json") + ": No such file or directory"
    if case == "no_complete":
        os.remove(os.path.join(path, "COMPLETE"))
        return "io_error", "Checkpoint is incomplete or manifest checksum failed"
    if case == "stale_complete":
        with open(os.path.join(path, "manifest.json"), "a") as f:
            f.write(" ")
        return "io_error", "Checkpoint is incomplete or manifest checksum failed"
    if case == "format":
        m["format"] = "mini-mla-weights"
        _resign(path, m)
        return "unsupported", "Unsupported model format or inference export used for resume"
    if case == "version":
        m["version"] = 2
        _resign(path, m)
        return "unsupported", "Unsupported model format or inference export used for resume"
    if case == "config_flag":
        with open(os.path.join(path, "config.json")) as f:
            c = json.load(f)
        c["bias"] = True
        with open(os.path.join(path, "config.json"), "w") as f:
            json.dump(c, f)
        return "unsupported", "Only v1 tied-embedding, bias-free MLA"
    if case == "config_hash":
        m["model_config_sha256"] = "0" * 64
        _resign(path, m)
        return "invalid_argument", "Checkpoint model configuration mismatch"
    if case == "parameter_count":
        m["parameter_count"] += 1
        _resign(path, m)
        return "invalid_argument", "Checkpoint model configuration mismatch"
    if case == "tokenizer_hash":
        m["tokenizer_sha256"] = "f" * 64
        _resign(path, m)
        return "invalid_argument", "Checkpoint tokenizer mismatch"
    if case == "tokenizer_vocab":
        tok = _tokenizer("mla36m")
        with open(os.path.join(path, "tokenizer.json"), "wb") as f:
            f.write(tok)
        m["tokenizer_sha256"] = hashlib.sha256(tok).hexdigest()
        _resign(path, m)
        return "invalid_argument", "Checkpoint tokenizer mismatch"
    if case == "tokenizer_specials":
        tok = json.loads(_tokenizer("tiny"))
        tok["specials"]["<|bos|>"] = 1
        raw = (json.dumps(tok, sort_keys=True, separators=(",", ":")) + "\n").encode()
        with open(os.path.join(path, "tokenizer.json"), "wb") as f:
            f.write(raw)
        return "invalid_argument", "Special token IDs disagree with the native chat template"
    if case == "file_name":
        m["sha256"]["../weights.bin"] = m["sha256"]["weights.bin"]
        _resign(path, m)
        return "io_error", "Invalid checkpoint filename"
    if case == "file_hash":
        _flip(path, "weights.bin", 100)
        return "io_error", "Checkpoint file checksum failed: weights.bin"
    if case == "tensor_file":
        t[3]["file"] = "weights2.bin"
        _resign(path, m)
        return "io_error", "Invalid tensor filename"
    if case == "duplicate":
        t.insert(4, dict(t[3]))
        _resign(path, m)
        return "io_error", "Duplicate named tensor"
    if case == "extent":
        t[5]["offset"] += 2
        _resign(path, m)
        return "io_error", "Invalid tensor extent or missing tensor file"
    if case == "crc":
        _flip(path, "weights.bin", t[6]["offset"])
        _resign(path, m)
        return "io_error", "Tensor checksum failed: " + t[6]["name"]
    if case == "unexpected":
        t[2]["name"] = "layers.0.attn.bias"
        _resign(path, m)
        return "io_error", "Unexpected tensor: layers.0.attn.bias"
    if case == "shape":
        t[3]["shape"] = t[3]["shape"][::-1]
        _resign(path, m)
        return "io_error", "Tensor shape, dtype, role, or file mismatch: " + t[3]["name"]
    if case == "role":
        t[2]["role"] = "hidden_matrix"
        _resign(path, m)
        return "io_error", "Tensor shape, dtype, role, or file mismatch: " + t[2]["name"]
    if case == "dtype":
        t[4]["dtype"] = "bf16"
        _resign(path, m)
        return "io_error", "Tensor shape, dtype, role, or file mismatch: " + t[4]["name"]
    if case == "nonfinite":
        e = t[7]
        with open(os.path.join(path, "weights.bin"), "r+b") as f:
            f.seek(e["offset"] + 8)
            f.write(struct.pack("<e", float("inf")) if e["dtype"] == "f16"
                    else struct.pack("<f", float("nan")))
            f.seek(e["offset"])
            e["crc32"] = zlib.crc32(f.read(e["nbytes"]))
        _resign(path, m)
        return "io_error", "Nonfinite checkpoint tensor: " + e["name"]
    if case == "missing":
        gone = t.pop()
        with open(os.path.join(path, "weights.bin"), "r+b") as f:
            f.truncate(gone["offset"])
        _resign(path, m)
        return "io_error", "Checkpoint is missing tensor: " + gone["name"]
    if case == "trailing":
        with open(os.path.join(path, "weights.bin"), "ab") as f:
            f.write(b"\0" * 4)
        _resign(path, m)
        return "io_error", "Unindexed trailing tensor data"
    raise AssertionError(case)


CASES = ["no_manifest", "no_complete", "stale_complete", "format", "version", "config_flag",
         "config_hash", "parameter_count", "tokenizer_hash", "tokenizer_vocab",
         "tokenizer_specials", "file_name", "file_hash", "tensor_file", "duplicate", "extent",
         "crc", "unexpected", "shape", "role", "dtype", "nonfinite", "missing", "trailing"]


@pytest.mark.parametrize("case", CASES)
def test_defective_exports_fail_like_the_reference(tmp_path, tiny_fixture, case):
    import cpp_inference_train_engine_amd as mla
    path = _write(tmp_path, TINY, tiny_fixture["params"], _tokenizer("tiny"), "f16")
    code, message = _corrupt(path, case)
    with pytest.raises(mla.MlaError) as e:
        mla.read_export(path)
    assert e.value.code == code, (e.value.code, str(e.value))
    assert message in str(e.value), str(e.value)


def test_missing_expected_tensor_is_named_in_sorted_order(tmp_path, tiny_fixture):
    """With several tensors absent the reference names the first in name order
    (expected.begin(), checkpoint.cpp:315-316)."""
    import cpp_inference_train_engine_amd as mla
    path = _write(tmp_path, TINY, tiny_fixture["params"], _tokenizer("tiny"), "f32")
    m = _manifest(path)
    kept = m["tensors"][:-3]
    dropped = sorted(e["name"] for e in m["tensors"][-3:])
    m["tensors"] = kept
    with open(os.path.join(path, "weights.bin"), "r+b") as f:
        f.truncate(kept[-1]["offset"] + kept[-1]["nbytes"])
    _resign(path, m)
    with pytest.raises(mla.MlaError) as e:
        mla.read_export(path)
    assert str(e.value).endswith("Checkpoint is missing tensor: " + dropped[0])


# ------------------------------------------------------------------ GPU ----
@pytest.mark.gpu
def test_engine_from_export_equals_engine_from_parameters(gpu, orc, tmp_path, tiny_fixture):
    """mla_engine_load of an f16 export of the reference's tiny-test weights gives the same
    logits as mla_engine_create with those weights (the device stores fp16 either way),
    and matches the oracle on the fp16-rounded weights."""
    params = tiny_fixture["params"]
    path = _write(tmp_path, TINY, params, _tokenizer("tiny"), "f16")
    loaded = gpu.HipEngine.load(path, max_sessions=2, max_rows=64, num_pages=16, page_size=16)
    direct = gpu.HipEngine(gpu.ModelConfig.from_dict(TINY), params, max_sessions=2,
                           max_rows=64, num_pages=16, page_size=16)
    prompt = tiny_fixture["tokens"]
    a, b = loaded.session(), direct.session()
    la, lb = a.prefill(prompt), b.prefill(prompt)
    np.testing.assert_array_equal(la, lb)
    for tok in (5, 17, 200):
        np.testing.assert_array_equal(a.decode(tok), b.decode(tok))
    ocfg = orc.Config.from_dict(TINY)
    p16 = params.astype(np.float16).astype(np.float32)
    want = orc.forward(ocfg, p16, list(prompt))[-1]
    assert np.abs(la - want).max() <= 5e-3
    model = gpu.HipModel.load(path, max_batch=4, page_size=16)
    assert model.cfg.vocab_size == 264
    model.close()
    loaded.close()
    direct.close()
