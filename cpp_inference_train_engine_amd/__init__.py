"""MI355X-native MLA cached-decode backend: Python binding of ``libmla_hip.so``.

The product is the C ABI declared in ``include/mla_hip.h`` (HIP kernels for
gfx950).  This module binds it with ctypes so tests and ``bench.py`` can drive
it with torch-allocated device buffers; torch is only plumbing for device
memory and streams.  There is no CPU fallback: every entry point raises when
the library is missing or a call fails.
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libmla_hip.so")

MLA_OK = 0
ERROR_NAMES = {1: "invalid_argument", 2: "io_error", 3: "unsupported", 4: "out_of_memory",
               5: "gpu_error", 6: "numerical_error", 7: "unavailable"}
DTYPE_F16, DTYPE_BF16 = 0, 1
WORK_DESC_INTS, WORK_PAGES, MAX_WORK, INFO_INTS = 8, 8, 65535, 8
DECODE_FORCE_GENERIC = 1
DECODE_FUSED_MERGE = 2
STEP_NO_READ_AHEAD = 4
DECODE_STATUS_XCD, DECODE_STATUS_UNPLACED = 1, 2
DECODE_WORKSPACE_HEAD, DECODE_STATUS_OFFSET = 1280, 1024
PLACE_MAX_SESSIONS = 256


class MlaError(RuntimeError):
    """A failed C-ABI call; ``code`` is the reference ErrorCode name."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.code = ERROR_NAMES.get(status, f"status{status}")
        super().__init__(f"{self.code}: {message}")


_lib = None

_SIGNATURES = {
    "mla_last_error": (C.c_char_p, []),
    "mla_abi_version": (C.c_int, []),
    "mla_build_metadata": (C.c_int, [C.c_void_p, C.c_int] + [C.c_void_p] * 4 +
                           [C.c_int] * 8 + [C.c_void_p] * 11),
    "mla_build_metadata_placed": (C.c_int, [C.c_void_p, C.c_int] + [C.c_void_p] * 4 +
                                  [C.c_int] * 8 + [C.c_void_p] * 11),
    "mla_xcd_placement_supported": (C.c_int, []),
    "mla_testing_fail_decode_status": (C.c_int, [C.c_int]),
    "mla_read_metadata_info": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "mla_decode_status": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]),
    "mla_append_latent": (C.c_int, [C.c_void_p] + [C.c_int] * 5 + [C.c_void_p] * 3 +
                          [C.c_int, C.c_void_p]),
    "mla_decode_workspace_bytes": (C.c_size_t, [C.c_int] * 4),
    "mla_decode_attention": (C.c_int, [C.c_void_p] + [C.c_int] * 6 + [C.c_float] +
                             [C.c_void_p] * 2 + [C.c_int] * 2 + [C.c_void_p] * 8 +
                             [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t,
                              C.c_int]),
    "mla_decode_partials": (C.c_int, [C.c_void_p] + [C.c_int] * 6 + [C.c_float] +
                            [C.c_void_p] * 2 + [C.c_int] * 2 + [C.c_void_p] * 8 +
                            [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t,
                             C.c_int]),
    "mla_decode_merge": (C.c_int, [C.c_void_p] + [C.c_int] * 3 + [C.c_void_p] * 4 +
                         [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    "mla_noalloc_scratch_bytes": (C.c_size_t, []),
    "mla_decode_attention_noalloc": (C.c_int, [C.c_void_p] + [C.c_int] * 6 + [C.c_float] +
                                     [C.c_void_p] * 2 + [C.c_int] * 2 + [C.c_void_p] * 8 +
                                     [C.c_int, C.c_void_p, C.c_void_p, C.c_int]),
    "mla_prefill_attention": (C.c_int, [C.c_void_p] + [C.c_int] * 6 + [C.c_float] +
                              [C.c_void_p] * 3 + [C.c_int] * 2 + [C.c_void_p] * 4 +
                              [C.c_int, C.c_void_p, C.c_void_p, C.c_int]),
    "mla_config_validate": (C.c_int, [C.c_void_p]),
    "mla_config_parameter_count": (C.c_size_t, [C.c_void_p]),
    "mla_model_create": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                   C.POINTER(C.c_void_p)]),
    "mla_model_destroy": (C.c_int, [C.c_void_p]),
    "mla_model_step": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int] + [C.c_void_p] * 4 +
                       [C.c_int, C.c_int] + [C.c_void_p] * 6 + [C.c_int] +
                       [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p, C.c_int]),
    "mla_model_logits": (C.c_void_p, [C.c_void_p]),
    "mla_model_forward": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p,
                                    C.c_int, C.c_int] + [C.c_void_p] * 3 + [C.c_int, C.c_int] +
                          [C.c_void_p] * 6 + [C.c_int] +
                          [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p, C.c_int]),
    "mla_engine_create": (C.c_int, [C.c_void_p, C.c_void_p] + [C.c_int] * 4 +
                          [C.POINTER(C.c_void_p)]),
    "mla_engine_destroy": (C.c_int, [C.c_void_p]),
    "mla_engine_info": (C.c_int, [C.c_void_p, C.c_void_p]),
    "mla_session_create": (C.c_int, [C.c_void_p, C.POINTER(C.c_int)]),
    "mla_session_fork": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_int)]),
    "mla_session_release": (C.c_int, [C.c_void_p, C.c_int]),
    "mla_session_length": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_int)]),
    "mla_session_prefill": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p]),
    "mla_session_decode": (C.c_int, [C.c_void_p, C.c_int, C.c_uint16, C.c_void_p]),
    "mla_engine_step": (C.c_int, [C.c_void_p, C.c_int] + [C.c_void_p] * 5),
    "mla_model_update_weights": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "mla_engine_update_weights": (C.c_int, [C.c_void_p, C.c_void_p]),
    "mla_engine_stats": (C.c_int, [C.c_void_p, C.c_void_p]),
    "mla_engine_forward": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "mla_export_read_config": (C.c_int, [C.c_char_p, C.c_void_p]),
    "mla_export_read": (C.c_int, [C.c_char_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    "mla_config_hash": (C.c_int, [C.c_void_p, C.c_char_p]),
    "mla_model_load": (C.c_int, [C.c_char_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "mla_engine_load": (C.c_int, [C.c_char_p] + [C.c_int] * 4 + [C.c_void_p, C.c_void_p]),
    "mla_tokenizer_load": (C.c_int, [C.c_char_p, C.c_void_p]),
    "mla_tokenizer_destroy": (C.c_int, [C.c_void_p]),
    "mla_tokenizer_info": (C.c_int, [C.c_void_p, C.c_void_p, C.c_char_p]),
    "mla_tokenizer_special": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p]),
    "mla_tokenizer_encode": (C.c_int, [C.c_void_p, C.c_char_p, C.c_size_t, C.c_int, C.c_void_p,
                                       C.c_size_t, C.c_void_p]),
    "mla_tokenizer_decode": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p,
                                       C.c_size_t, C.c_void_p]),
    "mla_model_set_banned": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "mla_engine_set_banned": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "mla_engine_config": (C.c_int, [C.c_void_p, C.c_void_p]),
    "mla_generation_config_init": (None, [C.c_void_p]),
    "mla_generation_config_validate": (C.c_int, [C.c_void_p]),
    "mla_sample_token": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p,
                                   C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "mla_tokenizer_banned": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "mla_generation_create": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_int,
                                        C.c_void_p, C.c_void_p, C.c_void_p]),
    "mla_generation_step": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "mla_generation_finished": (C.c_int, [C.c_void_p]),
    "mla_generation_result": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p,
                                        C.c_void_p, C.c_size_t, C.c_void_p, C.c_char_p]),
    "mla_generation_destroy": (C.c_int, [C.c_void_p]),
    "mla_scheduler_config_init": (None, [C.c_void_p]),
    "mla_scheduler_create": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "mla_scheduler_destroy": (C.c_int, [C.c_void_p]),
    "mla_scheduler_stop": (C.c_int, [C.c_void_p]),
    "mla_scheduler_submit": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_int,
                                       C.c_void_p]),
    "mla_scheduler_cancel": (C.c_int, [C.c_void_p, C.c_uint64]),
    "mla_scheduler_poll": (C.c_int, [C.c_void_p, C.c_uint64, C.c_int, C.c_void_p, C.c_size_t,
                                     C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "mla_scheduler_metrics_get": (C.c_int, [C.c_void_p, C.c_void_p]),
    "mla_scheduler_metrics_text": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
}


def lib() -> C.CDLL:
    """Load the HIP library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return sorted(_SIGNATURES)


def check(status: int) -> None:
    if status != MLA_OK:
        msg = lib().mla_last_error().decode(errors="replace")
        raise MlaError(status, msg)


def ptr(t) -> int | None:
    """Device (or host) address of a torch tensor / numpy array, None for None."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data


def stream_handle(stream=None) -> int | None:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


from .ops import (  # noqa: E402  (re-exported operator interface)
    PagedLatentCache, RaggedBatch, append_latent, build_metadata, decode_attention,
    decode_merge, decode_partials, decode_status, decode_workspace, decode_workspace_bytes,
    placed_work_slots, prefill_attention, xcd_count)
from . import ops  # noqa: E402

from .model import (HipModel, ModelConfig, config_hash, config_parameter_count,  # noqa: E402
                    config_validate, read_export)
from .engine import HipEngine, HipExecution, generate_tokens  # noqa: E402
from .tokenizer import HipTokenizer, clean_utf8  # noqa: E402
from .generation import (GenerationConfig, banned_tokens, generate,  # noqa: E402
                         generate_ids, sample_token)
from .scheduler import Scheduler  # noqa: E402

__all__ = ["MlaError", "lib", "check", "build_metadata", "append_latent", "decode_attention",
           "decode_partials", "decode_merge", "prefill_attention", "HipModel", "HipEngine",
           "HipExecution", "generate_tokens", "ModelConfig", "config_validate",
           "config_parameter_count", "config_hash", "read_export", "HipTokenizer",
           "clean_utf8", "generate", "generate_ids", "GenerationConfig", "sample_token",
           "banned_tokens", "Scheduler",
           "decode_workspace_bytes", "RaggedBatch", "PagedLatentCache", "DTYPE_F16",
           "DTYPE_BF16"]
