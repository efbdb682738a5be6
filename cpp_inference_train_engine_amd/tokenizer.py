"""The reference's tokenizer over the C ABI (``mla_tokenizer_*``, src/infer/tokenizer.cpp).

``HipTokenizer`` loads a ``mini-mla-tokenizer`` file with the reference's checks and
encodes (ranked byte-level BPE), decodes and builds chat prompts
(``Tokenizer::chat_prompt``, tokenizer.cpp:236-262); ``clean_utf8`` is the reference's
text cleaning (tokenizer.cpp:13-57).
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
        self._lib, self._h = lib(), h
        vocab = C.c_int()
        digest = C.create_string_buffer(65)
        check(lib().mla_tokenizer_info(h, C.byref(vocab), digest))
        self.vocab_size = vocab.value
        self.hash = digest.value.decode()

    def close(self):
        if getattr(self, "_h", None):
            self._lib.mla_tokenizer_destroy(self._h)  # kept at creation (interpreter exit)
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
