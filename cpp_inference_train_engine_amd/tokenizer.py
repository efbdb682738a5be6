"""Text in and out of the engine: the reference's tokenizer over the C ABI
(``mla_tokenizer_*``, src/infer/tokenizer.cpp) and greedy text generation
(``InferenceEngine::generate``, src/infer/inference.cpp:461-579).

``HipTokenizer`` loads a ``mini-mla-tokenizer`` file with the reference's checks and
encodes (ranked byte-level BPE), decodes and builds chat prompts
(``Tokenizer::chat_prompt``, tokenizer.cpp:236-262).  ``generate`` prefixes
``<|bos|>`` to the encoded prompt, runs the greedy generation loop with the reference's
stop rules (EOS, stop token sequences, stop strings) and returns the text cleaned as
``clean_utf8`` does (tokenizer.cpp:44-57).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import MlaError, check, lib

SPECIALS = ("<|pad|>", "<|bos|>", "<|eos|>", "<|user|>", "<|assistant|>", "<|system|>",
            "<|tool|>", "<|sep|>")


class HipTokenizer:
    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib().mla_tokenizer_load(os.fsencode(path), C.byref(h)))
        self._h = h
        vocab = C.c_int()
        digest = C.create_string_buffer(65)
        check(lib().mla_tokenizer_info(h, C.byref(vocab), digest))
        self.vocab_size = vocab.value
        self.hash = digest.value.decode()

    def close(self):
        if getattr(self, "_h", None):
            lib().mla_tokenizer_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def special(self, name: str) -> int:
        out = C.c_uint16()
        check(lib().mla_tokenizer_special(self._h, name.encode(), C.byref(out)))
        return out.value

    def encode(self, text, allow_special: bool = False) -> np.ndarray:
        raw = text.encode() if isinstance(text, str) else bytes(text)
        n = C.c_size_t()
        check(lib().mla_tokenizer_encode(self._h, raw, len(raw), int(allow_special), None, 0,
                                         C.byref(n)))
        ids = np.empty(n.value, np.uint16)
        check(lib().mla_tokenizer_encode(self._h, raw, len(raw), int(allow_special),
                                         ids.ctypes.data, ids.size, C.byref(n)))
        return ids

    def decode(self, ids, skip_special: bool = False) -> bytes:
        ids = np.ascontiguousarray(np.asarray(ids, np.uint16).ravel())
        n = C.c_size_t()
        check(lib().mla_tokenizer_decode(self._h, ids.ctypes.data, ids.size, int(skip_special),
                                         None, 0, C.byref(n)))
        buf = C.create_string_buffer(max(n.value, 1))
        check(lib().mla_tokenizer_decode(self._h, ids.ctypes.data, ids.size, int(skip_special),
                                         buf, n.value, C.byref(n)))
        return buf.raw[:n.value]

    def token_bytes(self, token: int) -> bytes:
        return self.decode([token])

    def chat_prompt(self, messages) -> list:
        """Tokenizer::chat_prompt (tokenizer.cpp:236-262): <|bos|>, then per message its
        role token, a newline, the content, <|eos|> and a newline; then <|assistant|> and
        a newline."""
        if not messages:
            raise MlaError(1, "Messages must not be empty")
        ids = [self.special("<|bos|>")]
        for m in messages:
            role, content = m["role"], m["content"]
            if role not in ("system", "user", "assistant", "tool"):
                raise MlaError(1, "Unsupported chat role")
            ids += [self.special(f"<|{role}|>"), 10]
            ids += self.encode(content).tolist()
            ids += [self.special("<|eos|>"), 10]
        return ids + [self.special("<|assistant|>"), 10]


def _utf8_length(b: bytes, i: int) -> int:
    """Length of the valid UTF-8 sequence at b[i], 0 when none (tokenizer.cpp:13-33)."""
    c = b[i]
    if c < 0x80:
        return 1
    n = 2 if 0xC2 <= c <= 0xDF else 3 if 0xE0 <= c <= 0xEF else 4 if 0xF0 <= c <= 0xF4 else 0
    if not n or i + n > len(b):
        return 0
    if any(not 0x80 <= b[i + k] <= 0xBF for k in range(1, n)):
        return 0
    d = b[i + 1]
    if (c == 0xE0 and d < 0xA0) or (c == 0xED and d >= 0xA0) or (c == 0xF0 and d < 0x90) or \
            (c == 0xF4 and d >= 0x90):
        return 0
    return n


def clean_utf8(b: bytes) -> str:
    """clean_utf8 (tokenizer.cpp:44-57): every byte that does not start a valid sequence
    becomes U+FFFD, one byte at a time."""
    out, i = bytearray(), 0
    while i < len(b):
        n = _utf8_length(b, i)
        if n:
            out += b[i:i + n]
            i += n
        else:
            out += "\ufffd".encode()
            i += 1
    return out.decode()


def generate(execution, tokenizer: HipTokenizer, prompt: str, max_new_tokens: int,
             max_sequence_length: int, stop=(), stop_tokens=()) -> dict:
    """InferenceEngine::generate + generate_tokens (inference.cpp:461-579), greedy: the
    prompt is <|bos|> + encode(prompt); generation stops at <|eos|>, at the end of a stop
    token sequence (its text removed) or at a stop string (text cut before it)."""
    ids = [tokenizer.special("<|bos|>")] + tokenizer.encode(prompt).tolist()
    if not ids or len(ids) + max_new_tokens > max_sequence_length:
        raise MlaError(1, "Prompt plus requested tokens exceeds context")
    for seq in stop_tokens:
        if any(t >= tokenizer.vocab_size for t in seq):
            raise MlaError(1, "Stop token exceeds vocabulary")
    eos = tokenizer.special("<|eos|>")
    logits = execution.prefill(ids)
    tokens, text, reason = [], b"", "length"
    for i in range(max_new_tokens):
        if not np.isfinite(logits).all():
            raise MlaError(6, "Invalid sampler logits")
        token = int(np.argmax(logits))  # the lowest index among the maxima
        tokens.append(token)
        if token == eos:
            reason = "stop"
            break
        hit = next((list(s) for s in stop_tokens
                    if len(tokens) >= len(s) and tokens[-len(s):] == list(s)), None)
        if hit is not None:
            text = tokenizer.decode(tokens, skip_special=True)
            tail = tokenizer.decode(hit, skip_special=True)
            if len(tail) <= len(text):
                text = text[:len(text) - len(tail)]
            reason = "stop"
            break
        text += tokenizer.token_bytes(token)
        found = next((text.find(s.encode()) for s in stop if text.find(s.encode()) >= 0), -1)
        if found >= 0:  # the first stop string of the list that occurs
            text = text[:found]
            reason = "stop"
            break
        if i + 1 < max_new_tokens:
            logits = execution.decode(token)
    return {"tokens": tokens, "text": clean_utf8(text), "finish_reason": reason,
            "prompt_tokens": len(ids)}
