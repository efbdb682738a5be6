"""Batched decode step over the C ABI (``mla_model_*`` in include/mla_hip.h).

``ModelConfig`` carries the fields of the reference's ``mini_mla::ModelConfig``
(include/mini_mla/model_config.hpp:5-19) and loads the same JSON keys
(src/model/config.cpp:77-115).  ``HipModel`` owns an uploaded model (fp16 weights
on the device) and runs one decode step for a batch of sessions: the
``CpuDecoder::decode`` math (src/infer/inference.cpp:76-173) for every session at
once, attention over the paged latent cache included.
"""
from __future__ import annotations

import ctypes as C
import json
import os

from . import DECODE_FUSED_MERGE, STEP_NO_READ_AHEAD, check, lib, ptr, stream_handle

_FIELDS = ("vocab_size", "max_sequence_length", "n_layers", "d_model", "n_heads",
           "head_dim_nope", "head_dim_rope", "head_dim_value", "q_lora_rank", "kv_lora_rank",
           "d_ff")


class ModelConfig(C.Structure):
    _fields_ = [(f, C.c_int) for f in _FIELDS] + [("norm_epsilon", C.c_float),
                                                   ("rope_theta", C.c_float)]

    @classmethod
    def from_dict(cls, d: dict) -> "ModelConfig":
        """The architecture keys of a reference config JSON (config/mla36m-v1.json)."""
        missing = [k for k in _FIELDS + ("norm_epsilon", "rope_theta") if k not in d]
        if missing:
            raise ValueError(f"config is missing {missing}")
        return cls(*[int(d[f]) for f in _FIELDS], float(d["norm_epsilon"]),
                   float(d["rope_theta"]))

    @classmethod
    def load(cls, path: str) -> "ModelConfig":
        with open(path) as f:
            return cls.from_dict(json.load(f))

    def to_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_}

    @property
    def qk_dim(self) -> int:
        return self.head_dim_nope + self.head_dim_rope


def config_validate(cfg: ModelConfig) -> None:
    """ModelConfig::validate (src/model/config.cpp:20-48); raises MlaError."""
    check(lib().mla_config_validate(C.byref(cfg)))


def config_hash(cfg: ModelConfig) -> str:
    """ModelConfig::hash (src/model/config.cpp:71-73): SHA-256 of the canonical JSON."""
    out = C.create_string_buffer(65)
    check(lib().mla_config_hash(C.byref(cfg), out))
    return out.value.decode()


def read_export(path: str):
    """load_checkpoint(path, training=false) (src/train/checkpoint.cpp:186-324) of a model
    export or checkpoint directory: (ModelConfig, fp32 parameters in registry order).
    Raises MlaError with the reference's code and message when a check fails."""
    import numpy as np
    cfg = ModelConfig()
    enc = os.fsencode(path)
    check(lib().mla_export_read_config(enc, C.byref(cfg)))
    params = np.empty(config_parameter_count(cfg), np.float32)
    check(lib().mla_export_read(enc, C.byref(cfg), params.ctypes.data, params.size))
    return cfg, params


def config_parameter_count(cfg: ModelConfig) -> int:
    """ModelConfig::parameter_count (src/model/config.cpp:7-19)."""
    return int(lib().mla_config_parameter_count(C.byref(cfg)))


class HipModel:
    """An uploaded model (mla_model_create): fp16 tiled weights and device activations
    for up to ``max_batch`` sessions per step."""

    def __init__(self, cfg: ModelConfig, params, max_batch: int, page_size: int = 64):
        import numpy as np
        params = np.ascontiguousarray(params, dtype=np.float32)
        if params.size != config_parameter_count(cfg):
            raise ValueError(f"expected {config_parameter_count(cfg)} parameters, got {params.size}")
        self.cfg, self.max_batch, self.page_size = cfg, max_batch, page_size
        h = C.c_void_p()
        check(lib().mla_model_create(C.byref(cfg), params.ctypes.data, max_batch, page_size,
                                     C.byref(h)))
        self._lib, self._h = lib(), h

    @classmethod
    def load(cls, path: str, max_batch: int, page_size: int = 64) -> "HipModel":
        """mla_model_load: a model export or checkpoint directory straight to the device."""
        self = cls.__new__(cls)
        self.cfg, self.max_batch, self.page_size = ModelConfig(), max_batch, page_size
        h = C.c_void_p()
        check(lib().mla_model_load(os.fsencode(path), max_batch, page_size, C.byref(self.cfg),
                                   C.byref(h)))
        self._lib, self._h = lib(), h
        return self

    def update_weights(self, params) -> int:
        """mla_model_update_weights: new weights in place (Model::mark_weights_changed);
        returns the revision count.  No step may be in flight."""
        import numpy as np
        params = np.ascontiguousarray(params, dtype=np.float32)
        if params.size != config_parameter_count(self.cfg):
            raise ValueError(f"expected {config_parameter_count(self.cfg)} parameters, got {params.size}")
        rev = C.c_uint64()
        check(lib().mla_model_update_weights(self._h, params.ctypes.data, C.byref(rev)))
        return rev.value

    def close(self):
        # The library handle kept at creation: at interpreter exit the package's
        # globals may already be cleared when this runs.
        if getattr(self, "_h", None):
            self._lib.mla_model_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def step(self, batch, tokens, positions, pages, workspace, logits=None, next_tokens=None,
             stream=None, read_ahead=True):
        """One decode step.  ``batch`` is the RaggedBatch of mla_build_metadata (q_len = 1,
        ctx_len = positions); ``pages`` is the list of per-layer page pools; tokens and
        positions are device int32 [B].  read_ahead=False turns off the L2 read-ahead of
        the attention's pages (MLA_STEP_NO_READ_AHEAD: same results, other timing).
        Returns (logits [B x vocab] fp32, next_tokens [B])."""
        import torch
        B = int(tokens.numel())
        dev = tokens.device
        if logits is None:
            logits = torch.empty((B, self.cfg.vocab_size), dtype=torch.float32, device=dev)
        if next_tokens is None:
            next_tokens = torch.empty(B, dtype=torch.int32, device=dev)
        pools = (C.c_void_p * self.cfg.n_layers)(*[p.data_ptr() for p in pages])
        check(lib().mla_model_step(
            self._h, stream_handle(stream), B, ptr(tokens), ptr(positions),
            ptr(batch.cu_seqlens_q), ptr(batch.page_table), batch.max_pages,
            batch.num_pool_pages, ptr(batch.slot_mapping), ptr(batch.num_splits),
            ptr(batch.cu_splits), ptr(batch.work_desc), ptr(batch.work_pages), ptr(batch.info),
            batch.max_work, pools, ptr(workspace), int(workspace.numel()), ptr(logits),
            ptr(next_tokens),
            (DECODE_FUSED_MERGE if batch.placed else 0) | (0 if read_ahead else STEP_NO_READ_AHEAD)))
        return logits, next_tokens
