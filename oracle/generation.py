"""Test infrastructure, not product code: a pure-Python restatement of the reference's
token selection and generation loop, the checker for the library's ``mla_sample_token``
and ``mla_generation_*`` (used only by tests/).

Restated from the reference (file:line):
  * ``Rng`` (include/mini_mla/rng.hpp:9-19): SplitMix64; uniform = (top 24 bits + 0.5)/2^24;
  * ``GenerationConfig::validate`` (src/infer/inference.cpp:330-344);
  * ``sample_token`` (src/infer/inference.cpp:345-412): greedy over the ids not banned with
    the repetition penalty on history ids (strict >, lowest id wins); otherwise penalise
    each history id once, drop banned ids, order by score then id, keep top_k, the
    smallest prefix whose mass reaches top_p of the total, draw u * kept and walk down;
  * ``utf8_length`` / ``clean_utf8`` (src/infer/tokenizer.cpp:13-57), ``stream_prefix``
    (inference.cpp:253-263);
  * ``generate_tokens`` (inference.cpp:469-579), over an execution given as two
    callables.

Scores are float32 as in the reference (np.float32 arithmetic for the penalty and the
score difference); probabilities, their sum and the draw are Python floats (doubles),
as the reference's are.  Pinned in tests/test_generation.py against the reference's own
sampler test (tests/test_training.cpp:77-110), closed-form draws on small
distributions and empirical frequencies over many seeded draws.
"""
from __future__ import annotations

import math

import numpy as np

M64 = (1 << 64) - 1


class Rng:
    def __init__(self, seed: int = 42):
        self.state = seed & M64

    def next(self) -> int:
        self.state = (self.state + 0x9E3779B97F4A7C15) & M64
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> 31)

    def uniform(self) -> float:
        return float((np.float32(self.next() >> 40) + np.float32(0.5)) / np.float32(16777216.0))


class SettingsError(ValueError):
    pass


def validate(cfg: dict) -> None:
    t, p, rp = cfg["temperature"], cfg["top_p"], cfg["repetition_penalty"]
    if (cfg["max_new_tokens"] < 0 or cfg["max_new_tokens"] > 65535 or cfg["top_k"] < 0 or
            not math.isfinite(t) or t < 0 or not math.isfinite(p) or p <= 0 or p > 1 or
            not math.isfinite(rp) or rp <= 0):
        raise SettingsError("Invalid generation settings")
    for s in cfg.get("stop", ()):
        if not s or len(s) > 4096:
            raise SettingsError("Stop strings must be nonempty and <=4096 bytes")
    for s in cfg.get("stop_tokens", ()):
        if not s:
            raise SettingsError("Stop token sequences must be nonempty")


def _penalised(score, rp):
    score, rp = np.float32(score), np.float32(rp)
    return score / rp if score > 0 else score * rp


def sample_token(logits, history, cfg: dict, rng: Rng, banned=()) -> int:
    validate(cfg)
    logits = [np.float32(x) for x in logits]
    if not logits or len(logits) > 65535 or not all(math.isfinite(x) for x in logits):
        raise ArithmeticError("Invalid sampler logits")
    V, rp = len(logits), np.float32(cfg["repetition_penalty"])
    if cfg["temperature"] == 0:
        ban = {b for b in banned if b < V}
        rep = {h for h in history if h < V} if rp != 1 else set()
        best, top = None, None
        for i in range(V):
            if i in ban:
                continue
            s = _penalised(logits[i], rp) if i in rep else logits[i]
            if best is None or s > top:
                best, top = i, s
        if best is None:
            raise SettingsError("All tokens are banned")
        return best
    score = list(logits)
    if rp != 1:
        seen = set()
        for h in history:
            if h < V and h not in seen:
                seen.add(h)
                score[h] = _penalised(score[h], rp)
    for b in banned:
        if b < V:
            score[b] = np.float32(-np.inf)
    order = [i for i in range(V) if math.isfinite(score[i])]
    if not order:
        raise SettingsError("All tokens are banned")
    order.sort(key=lambda i: (-float(score[i]), i))
    if 0 < cfg["top_k"] < len(order):
        order = order[:cfg["top_k"]]
    temp = float(np.float32(cfg["temperature"]))
    prob = [math.exp(float(np.float32(score[i] - score[order[0]])) / temp) for i in order]
    total = 0.0
    for p in prob:
        total += p
    kept, count = 0.0, 0
    while True:
        kept += prob[count]
        count += 1
        if not (count < len(order) and kept < float(np.float32(cfg["top_p"])) * total):
            break
    draw = rng.uniform() * kept
    for i in range(count):
        draw -= prob[i]
        if draw <= 0:
            return order[i]
    return order[count - 1]


def utf8_length(b: bytes, i: int) -> int:
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


def clean_utf8(b: bytes) -> bytes:
    out, i = bytearray(), 0
    while i < len(b):
        n = utf8_length(b, i)
        if n:
            out += b[i:i + n]
            i += n
        else:
            out += b"\xef\xbf\xbd"
            i += 1
    return bytes(out)


def stream_prefix(s: bytes, limit: int) -> int:
    i = 0
    while i < limit:
        c = s[i]
        n = 1 if c < 0xC0 else 2 if c < 0xE0 else 3 if c < 0xF0 else 4 if c <= 0xF4 else 1
        if i + n > limit:
            break
        i += n
    return i


def banned_ids(token_bytes: list, eos: int) -> list:
    """InferenceEngine::load (inference.cpp:441-447): specials (the last eight ids) other
    than eos, and ids without bytes."""
    V = len(token_bytes)
    return [i for i in range(V) if (i >= V - 8 and i != eos) or not token_bytes[i]]


def generate_tokens(prefill, decode, token_bytes: list, eos: int, prompt, cfg: dict,
                    max_sequence_length: int, callback=None) -> dict:
    """generate_tokens (inference.cpp:469-579).  token_bytes[i]: the bytes of id i (b"" for
    unassigned ids, the spelling for specials); specials are the last eight ids."""
    validate(cfg)
    if not prompt or len(prompt) + cfg["max_new_tokens"] > max_sequence_length:
        raise SettingsError("Prompt plus requested tokens exceeds context")
    V = len(token_bytes)

    def decode_text(ids, skip_special):
        out = b""
        for i in ids:
            if i >= V or not token_bytes[i]:
                raise SettingsError("Unknown token ID")
            if not (skip_special and i >= V - 8):
                out += token_bytes[i]
        return out

    stop = [s.encode() if isinstance(s, str) else s for s in cfg.get("stop", ())]
    stop_tokens = [list(s) for s in cfg.get("stop_tokens", ())]
    hold = max([len(s) for s in stop] + [0])
    for seq in stop_tokens:
        if any(t >= V for t in seq):
            raise SettingsError("Stop token exceeds vocabulary")
        hold = max(hold, sum(len(token_bytes[t]) for t in seq))
    banned = banned_ids(token_bytes, eos)
    logits = prefill(list(prompt))
    history, rng = list(prompt), Rng(cfg["seed"])
    tokens, text, reason, emitted = [], b"", "length", 0
    for i in range(cfg["max_new_tokens"]):
        if callback and not callback(b""):
            reason = "cancelled"
            break
        token = sample_token(logits, history, cfg, rng, banned)
        tokens.append(token)
        history.append(token)
        if token == eos:
            reason = "stop"
            break
        hit = next((s for s in stop_tokens if len(tokens) >= len(s) and tokens[-len(s):] == s),
                   None)
        if hit is not None:
            text = decode_text(tokens, True)
            tail = decode_text(hit, True)
            if len(tail) <= len(text):
                text = text[:len(text) - len(tail)]
            reason = "stop"
            break
        text += token_bytes[token]
        stopped = False
        for s in stop:
            p = text.find(s)
            if p >= 0:
                text, reason, stopped = text[:p], "stop", True
                break
        limit = len(text) if stopped else max(len(text) - hold, 0)
        safe = stream_prefix(text, limit)
        if callback and safe > emitted:
            if not callback(clean_utf8(text[emitted:safe])):
                reason = "cancelled"
                break
            emitted = safe
        if stopped:
            break
        if i + 1 < cfg["max_new_tokens"]:
            logits = decode(token)
    if callback and reason != "cancelled" and len(text) > emitted and \
            not callback(clean_utf8(text[emitted:])):
        reason = "cancelled"
    return {"tokens": tokens, "text": clean_utf8(text).decode(), "finish_reason": reason}
