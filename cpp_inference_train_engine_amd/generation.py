"""Token selection and text generation over the C ABI (``mla_sample_token``,
``mla_generation_*``): the reference's ``GenerationConfig``, ``sample_token`` and
``InferenceEngine::generate`` / ``generate_tokens`` (src/infer/inference.cpp:330-579).

``generate`` prefixes ``<|bos|>`` to the encoded prompt; ``generate_ids`` takes ids.  Both
prefill through the execution, then hand each set of logits to the library's generation
state machine, which samples (greedy or seeded temperature / top-k / top-p, with the
repetition penalty and the tokenizer's banned ids), applies the stop rules (EOS, stop
token sequences, stop strings), streams text through ``callback`` (return False to
cancel) and names the token to decode next.
"""
from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass, field

import numpy as np

from . import MlaError, check, lib


@dataclass
class GenerationConfig:
    """GenerationConfig (include/mini_mla/inference.hpp:27-34), same defaults."""
    max_new_tokens: int = 128
    top_k: int = 0
    temperature: float = 0.8
    top_p: float = 0.95
    repetition_penalty: float = 1.0
    seed: int = 42
    stop: tuple = field(default_factory=tuple)         # stop strings
    stop_tokens: tuple = field(default_factory=tuple)  # stop token sequences


class CGenerationConfig(C.Structure):
    _fields_ = [("max_new_tokens", C.c_int), ("top_k", C.c_int), ("temperature", C.c_float),
                ("top_p", C.c_float), ("repetition_penalty", C.c_float), ("seed", C.c_uint64),
                ("n_stop", C.c_int), ("stop", C.POINTER(C.c_char_p)),
                ("stop_len", C.POINTER(C.c_size_t)), ("n_stop_tokens", C.c_int),
                ("stop_tokens_len", C.POINTER(C.c_int)),
                ("stop_tokens", C.POINTER(C.c_uint16))]


def c_config(cfg: GenerationConfig | None, max_new_tokens_default: bool = False):
    """The C struct for cfg (None: the reference's defaults) and the buffers it points
    into, which the caller keeps alive for as long as the struct is used."""
    cfg = cfg if cfg is not None else GenerationConfig()
    c = CGenerationConfig()
    c.max_new_tokens = -1 if max_new_tokens_default else int(cfg.max_new_tokens)
    c.top_k, c.temperature, c.top_p = int(cfg.top_k), float(cfg.temperature), float(cfg.top_p)
    c.repetition_penalty, c.seed = float(cfg.repetition_penalty), int(cfg.seed) & (2**64 - 1)
    stops = [s.encode() if isinstance(s, str) else bytes(s) for s in cfg.stop]
    seqs = [[int(t) for t in seq] for seq in cfg.stop_tokens]
    if any(t < 0 or t > 65535 for seq in seqs for t in seq):
        raise MlaError(1, "Stop token exceeds vocabulary")
    keep = [(C.c_char_p * max(len(stops), 1))(*stops),
            (C.c_size_t * max(len(stops), 1))(*[len(s) for s in stops]),
            (C.c_int * max(len(seqs), 1))(*[len(s) for s in seqs]),
            (C.c_uint16 * max(sum(map(len, seqs)), 1))(*[t for s in seqs for t in s])]
    c.n_stop, c.stop, c.stop_len = len(stops), keep[0], keep[1]
    c.n_stop_tokens, c.stop_tokens_len, c.stop_tokens = len(seqs), keep[2], keep[3]
    return c, keep


def sample_token(logits, history=(), config: GenerationConfig | None = None,
                 rng_state: int | None = None, banned=()):
    """sample_token (inference.cpp:345-412) in the library: returns (token, rng_state)
    where rng_state is the Rng state after the draw (start: the config's seed)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32).ravel()
    history = np.ascontiguousarray(history, dtype=np.uint16).ravel()
    banned = np.ascontiguousarray(banned, dtype=np.uint16).ravel()
    cfg = config if config is not None else GenerationConfig()
    c, keep = c_config(cfg)
    state = C.c_uint64(cfg.seed if rng_state is None else rng_state)
    token = C.c_uint16()
    check(lib().mla_sample_token(logits.ctypes.data, logits.size, history.ctypes.data,
                                 history.size, C.byref(c), C.byref(state), banned.ctypes.data,
                                 banned.size, C.byref(token)))
    del keep
    return token.value, state.value


def banned_tokens(tokenizer) -> list:
    """The ids InferenceEngine::load bans (inference.cpp:441-447)."""
    n = C.c_size_t()
    check(lib().mla_tokenizer_banned(tokenizer._h, None, 0, C.byref(n)))
    out = np.empty(max(n.value, 1), np.uint16)
    check(lib().mla_tokenizer_banned(tokenizer._h, out.ctypes.data, out.size, C.byref(n)))
    return out[:n.value].tolist()


_TEXT_CALLBACK = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_void_p, C.c_size_t)


def generate(execution, tokenizer, prompt, config: GenerationConfig | None = None,
             max_sequence_length: int | None = None, callback=None) -> dict:
    """InferenceEngine::generate (inference.cpp:461-468): <|bos|> + encode(prompt)."""
    ids = [tokenizer.special("<|bos|>")] + tokenizer.encode(prompt).tolist()
    return generate_ids(execution, tokenizer, ids, config, max_sequence_length, callback)


def generate_ids(execution, tokenizer, ids, config: GenerationConfig | None = None,
                 max_sequence_length: int | None = None, callback=None) -> dict:
    """InferenceEngine::generate_tokens (inference.cpp:469-579) over any execution with
    ``prefill(ids) -> logits`` and ``decode(token) -> logits``.  Returns tokens, text,
    finish_reason, prompt_tokens and the timings (ms) the reference reports."""
    if max_sequence_length is None:
        max_sequence_length = execution.max_sequence_length
    ids = np.ascontiguousarray(ids, dtype=np.uint16).ravel()
    c, keep = c_config(config)
    failure = []

    def relay(_user, text, n):
        try:
            return int(bool(callback(C.string_at(text, n).decode())))
        except Exception as e:  # an exception in the callback cancels, then re-raises
            failure.append(e)
            return 0

    cb = _TEXT_CALLBACK(relay) if callback is not None else None
    h = C.c_void_p()
    check(lib().mla_generation_create(tokenizer._h, C.byref(c), ids.ctypes.data, ids.size,
                                      int(max_sequence_length),
                                      C.cast(cb, C.c_void_p) if cb else None, None, C.byref(h)))
    try:
        started = time.perf_counter()
        logits = execution.prefill(ids.tolist())
        result = {"prompt_tokens": int(ids.size), "decode_ms": 0.0, "time_to_first_token_ms": 0.0,
                  "prefill_ms": (time.perf_counter() - started) * 1e3}
        nxt, first = C.c_int32(-1), True
        while not lib().mla_generation_finished(h):
            logits = np.ascontiguousarray(logits, dtype=np.float32).ravel()
            check(lib().mla_generation_step(h, logits.ctypes.data, logits.size, C.byref(nxt)))
            if first:
                result["time_to_first_token_ms"] = (time.perf_counter() - started) * 1e3
                first = False
            if nxt.value < 0:
                break
            t = time.perf_counter()
            logits = execution.decode(nxt.value)
            result["decode_ms"] += (time.perf_counter() - t) * 1e3
        n_text, n_tok = C.c_size_t(), C.c_size_t()
        reason = C.create_string_buffer(16)
        check(lib().mla_generation_result(h, None, 0, C.byref(n_text), None, 0, C.byref(n_tok),
                                          reason))
        text = C.create_string_buffer(max(n_text.value, 1))
        tokens = np.empty(max(n_tok.value, 1), np.uint16)
        check(lib().mla_generation_result(h, text, n_text.value, C.byref(n_text),
                                          tokens.ctypes.data, tokens.size, C.byref(n_tok), reason))
    finally:
        lib().mla_generation_destroy(h)
        del keep
    if failure:
        raise failure[0]
    result.update(tokens=tokens[:n_tok.value].tolist(),
                  text=text.raw[:n_text.value].decode(), finish_reason=reason.value.decode())
    return result
