"""Session-level inference over the C ABI (``mla_engine_*`` / ``mla_session_*``).

``HipEngine`` owns an uploaded model and a paged latent cache shared by many sessions.
``HipExecution`` is one session with the reference's inference interface
(``mini_mla::Execution``, include/mini_mla/execution.hpp:28-62): ``prefill(ids)``
restarts the session and returns the last position's logits, ``decode(token)``
appends one token and returns its logits, ``fork_inference()`` opens a new empty
session on the same weights.  ``step`` batches several sessions into one GPU forward
(continuous batching, chunked prefill).  ``generate_tokens`` is the greedy path of
``InferenceEngine::generate_tokens`` (src/infer/inference.cpp:469-579).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import MlaError, check, lib
from .model import ModelConfig, config_parameter_count


class HipEngine:
    """mla_engine_create: one model, ``num_pages`` cache pages of ``page_size`` tokens per
    layer, up to ``max_sessions`` sessions and ``max_rows`` new tokens per step."""

    def __init__(self, cfg: ModelConfig, params, max_sessions: int = 16, max_rows: int = 1024,
                 num_pages: int = 1024, page_size: int = 64):
        params = np.ascontiguousarray(params, dtype=np.float32)
        if params.size != config_parameter_count(cfg):
            raise ValueError(f"expected {config_parameter_count(cfg)} parameters, got {params.size}")
        self.cfg = cfg
        h = C.c_void_p()
        check(lib().mla_engine_create(C.byref(cfg), params.ctypes.data, max_sessions, max_rows,
                                      num_pages, page_size, C.byref(h)))
        self._lib, self._h = lib(), h

    @classmethod
    def load(cls, path: str, max_sessions: int = 16, max_rows: int = 1024,
             num_pages: int = 1024, page_size: int = 64) -> "HipEngine":
        """mla_engine_load: an engine over a model export or checkpoint directory
        (load_checkpoint(path, training=false), src/train/checkpoint.cpp:186-324)."""
        self = cls.__new__(cls)
        self.cfg = ModelConfig()
        h = C.c_void_p()
        check(lib().mla_engine_load(os.fsencode(path), max_sessions, max_rows, num_pages,
                                    page_size, C.byref(self.cfg), C.byref(h)))
        self._lib, self._h = lib(), h
        return self

    @property
    def handle(self):
        if not self._h:
            raise MlaError(1, "engine is closed")
        return self._h

    def close(self):
        # Schedulers running on this engine stop first: their threads use it.
        for dependent in list(getattr(self, "_dependents", ())):
            dependent.close()
        if getattr(self, "_h", None):
            self._lib.mla_engine_destroy(self._h)  # kept at creation (interpreter exit)
            self._h = None

    def _attach(self, dependent) -> None:
        import weakref
        if not hasattr(self, "_dependents"):
            self._dependents = weakref.WeakSet()
        self._dependents.add(dependent)

    def __del__(self):
        self.close()

    def info(self) -> dict:
        v = (C.c_int64 * 8)()
        check(lib().mla_engine_info(self.handle, v))
        keys = ("active_sessions", "free_pages", "pages", "page_size", "max_rows",
                "max_sessions", "steps", "pool_bytes")
        return dict(zip(keys, [int(x) for x in v]))

    def session(self) -> "HipExecution":
        """A new empty session (Execution::fork_inference semantics)."""
        s = C.c_int()
        check(lib().mla_session_create(self.handle, C.byref(s)))
        return HipExecution(self, s.value)

    def set_banned(self, ids) -> None:
        """mla_engine_set_banned: the ids the greedy next tokens of later steps skip
        (sample_token's banned list, inference.cpp:345-380)."""
        ids = np.ascontiguousarray(ids, dtype=np.uint16).ravel()
        check(lib().mla_engine_set_banned(self.handle, ids.ctypes.data, ids.size))

    def update_weights(self, params) -> None:
        """mla_engine_update_weights: replace the weights (Model::mark_weights_changed);
        sessions with cached tokens must prefill again before they decode."""
        params = np.ascontiguousarray(params, dtype=np.float32)
        if params.size != config_parameter_count(self.cfg):
            raise ValueError(f"expected {config_parameter_count(self.cfg)} parameters, "
                             f"got {params.size}")
        check(lib().mla_engine_update_weights(self.handle, params.ctypes.data))

    def stats(self) -> dict:
        """mla_engine_stats: Execution::stats's counters (execution.hpp:25-27), engine-wide."""
        v = (C.c_uint64 * 6)()
        check(lib().mla_engine_stats(self.handle, v))
        keys = ("graph_submissions", "host_waits", "kernel_submissions", "copies", "revision",
                "fused_reruns")
        return dict(zip(keys, [int(x) for x in v]))

    def forward(self, ids, batch: int, sequence: int) -> np.ndarray:
        """mla_engine_forward: Execution::forward(ids, batch, sequence) (execution.hpp:
        38-39), the logits of every position, [batch * sequence, vocab]."""
        ids = np.ascontiguousarray(np.asarray(ids, np.uint16).ravel())
        if ids.size != batch * sequence:
            raise ValueError("ids must hold batch * sequence tokens")
        out = np.empty((batch * sequence, self.cfg.vocab_size), np.float32)
        check(lib().mla_engine_forward(self.handle, int(batch), int(sequence), ids.ctypes.data,
                                       out.ctypes.data))
        return out

    def step(self, sessions, token_lists, want_logits: bool = True):
        """One batched forward: ``sessions[i]`` appends ``token_lists[i]`` (one token =
        decode, several = chunked prefill).  Returns (logits [n, vocab] or None,
        greedy next tokens [n])."""
        n = len(sessions)
        ids = np.array([s.session_id for s in sessions], np.int32)
        counts = np.array([len(t) for t in token_lists], np.int32)
        toks = np.ascontiguousarray(np.concatenate([np.asarray(t, np.uint16).ravel()
                                                    for t in token_lists]), np.uint16)
        logits = np.empty((n, self.cfg.vocab_size), np.float32) if want_logits else None
        nxt = np.empty(n, np.int32)
        check(lib().mla_engine_step(self.handle, n, ids.ctypes.data, counts.ctypes.data,
                                    toks.ctypes.data,
                                    logits.ctypes.data if want_logits else None,
                                    nxt.ctypes.data))
        return logits, nxt


class HipExecution:
    """One session: the inference part of mini_mla::Execution on the HIP backend."""

    def __init__(self, engine: HipEngine, session_id: int):
        self.engine, self.session_id = engine, session_id
        self._logits = np.empty(engine.cfg.vocab_size, np.float32)

    def device_name(self) -> str:
        return "HIP / MI355X (gfx950)"

    def attention_name(self) -> str:
        return "paged-mla"

    def stats(self) -> dict:
        """Execution::stats: the engine's counters (its sessions share one stream)."""
        return self.engine.stats()

    def forward(self, ids, batch: int, sequence: int) -> np.ndarray:
        """Execution::forward: every position's logits, [batch * sequence, vocab]."""
        return self.engine.forward(ids, batch, sequence)

    def fork_inference(self) -> "HipExecution":
        """A new empty session on the same weights (execution.hpp:34-37)."""
        return self.engine.session()

    def fork_prefix(self) -> "HipExecution":
        """A new session holding this session's cached tokens (shared pages)."""
        s = C.c_int()
        check(lib().mla_session_fork(self.engine.handle, self.session_id, C.byref(s)))
        return HipExecution(self.engine, s.value)

    @property
    def max_sequence_length(self) -> int:
        return self.engine.cfg.max_sequence_length

    @property
    def position(self) -> int:
        n = C.c_int()
        check(lib().mla_session_length(self.engine.handle, self.session_id, C.byref(n)))
        return n.value

    def prefill(self, ids) -> np.ndarray:
        """CpuDecoder::prefill (inference.cpp:47-68): logits of the last prompt position."""
        ids = np.ascontiguousarray(np.asarray(ids, np.uint16).ravel())
        check(lib().mla_session_prefill(self.engine.handle, self.session_id, ids.ctypes.data,
                                        int(ids.size), self._logits.ctypes.data))
        return self._logits.copy()

    def decode(self, token: int) -> np.ndarray:
        """CpuDecoder::decode (inference.cpp:69-174): logits after appending ``token``."""
        check(lib().mla_session_decode(self.engine.handle, self.session_id, int(token),
                                       self._logits.ctypes.data))
        return self._logits.copy()

    def release(self):
        if self.session_id is not None and self.engine._h:
            check(lib().mla_session_release(self.engine.handle, self.session_id))
        self.session_id = None


def greedy_token(logits: np.ndarray) -> int:
    """sample_token with temperature 0, no bans or penalty (inference.cpp:354-380): the
    lowest index among the maxima (strict >); non-finite logits are an error."""
    if not np.isfinite(logits).all():
        raise MlaError(6, "Invalid sampler logits")
    return int(np.argmax(logits))


def generate_tokens(execution, prompt, max_new_tokens: int, max_sequence_length: int):
    """Greedy InferenceEngine::generate_tokens (inference.cpp:469-579): prefill, then per
    new token sample and, unless it is the last one, decode it.  Returns the tokens."""
    prompt = list(prompt)
    if not prompt or len(prompt) + max_new_tokens > max_sequence_length:
        raise MlaError(1, "Prompt plus requested tokens exceeds context")
    logits = execution.prefill(prompt)
    out = []
    for i in range(max_new_tokens):
        token = greedy_token(logits)
        out.append(token)
        if i + 1 < max_new_tokens:
            logits = execution.decode(token)
    return out
