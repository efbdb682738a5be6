"""Token selection and the generation loop (mla_sample_token, mla_generation_*,
GenerationConfig, generate / generate_ids) against oracle/generation.py, a Python
restatement of sample_token and generate_tokens (src/infer/inference.cpp:330-579).

The oracle is pinned first: the reference's own sampler test (tests/test_training.cpp:
77-110), its Rng against the C oracle's (itself pinned to the reference's rng.hpp), its
greedy rule against orc_greedy, draws on equal-probability ids where the chosen id is
fixed by the uniform alone, and empirical frequencies over many seeded draws against
softmax(logits / T) cut to the top-p nucleus.  The library's sampler must then return
the same id and leave the same Rng state as the oracle, and its generation loop the
same tokens, text, finish reason and streamed chunks.  Host code: CPU tests.
"""
import json
import math
import os

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import generation as og

TOK_TINY = os.path.join(GOLDEN, "tokenizer_tiny.json")


def cfg(**kw):
    base = dict(max_new_tokens=128, top_k=0, temperature=0.8, top_p=0.95, repetition_penalty=1.0,
                seed=42, stop=(), stop_tokens=())
    base.update(kw)
    return base


def gen_config(c):
    import cpp_inference_train_engine_amd as mla
    return mla.GenerationConfig(**c)


# ------------------------------------------------------- oracle pinning ----
def test_oracle_reference_sampler_test():
    """tests/test_training.cpp:77-110, verbatim in meaning."""
    scores = [2, -1, 1, 0]
    rng = og.Rng(1)
    assert og.sample_token(scores, [], cfg(temperature=0), rng) == 0
    assert og.sample_token(scores, [0, 0], cfg(temperature=0, repetition_penalty=3), rng) == 2
    for _ in range(30):
        assert og.sample_token(scores, [], cfg(temperature=0.7, top_k=1), rng) == 0
    a, b = og.Rng(99), og.Rng(99)
    c = cfg(temperature=0.7, top_p=1)
    for _ in range(50):
        assert og.sample_token(scores, [], c, a) == og.sample_token(scores, [], c, b)
    with pytest.raises(og.SettingsError):
        og.sample_token(scores, [], c, rng, [0, 1, 2, 3])
    with pytest.raises(og.SettingsError):
        og.sample_token(scores, [], cfg(temperature=0.7, top_p=0), rng)


def test_oracle_rng_is_the_reference_rng(orc):
    for seed in (0, 1, 42, 2**63 + 5):
        mine, theirs = og.Rng(seed), orc.Rng(seed)
        for _ in range(64):
            assert mine.next() == theirs.next()
        for _ in range(64):
            assert mine.uniform() == theirs.uniform()


def test_oracle_greedy_is_orc_greedy(orc):
    rng = np.random.default_rng(3)
    L = orc.lib()
    for _ in range(200):
        V = int(rng.integers(2, 40))
        logits = np.round(rng.normal(size=V), 1).astype(np.float32)  # ties happen
        hist = rng.integers(0, V + 3, int(rng.integers(0, 6))).astype(np.uint16)
        ban = rng.integers(0, V + 3, int(rng.integers(0, 4))).astype(np.uint16)
        rp = float(rng.choice([1.0, 1.5, 0.5]))
        want = L.orc_greedy(logits.ctypes.data, V, hist.ctypes.data, hist.size,
                            np.float32(rp), ban.ctypes.data, ban.size)
        try:
            got = og.sample_token(logits, hist.tolist(), cfg(temperature=0, repetition_penalty=rp),
                                  og.Rng(0), ban.tolist())
        except og.SettingsError:
            got = -1
        assert got == want


def test_oracle_equal_scores_follow_the_uniform():
    """Equal scores: every probability is exp(0) = 1, so the id is fixed by the draw
    alone: u * kept falls in [0,1] -> first id, (1,2] -> second, ... (ids in order)."""
    for seed in range(300):
        u = og.Rng(seed).uniform()
        got = og.sample_token([0.5] * 3, [], cfg(temperature=1.3, top_p=1.0), og.Rng(seed))
        assert got == (0 if u * 3 <= 1 else 1 if u * 3 <= 2 else 2)
        # top_p 0.5: kept grows 1 (< 1.5, go on), 2 (stop): the first two ids only
        got = og.sample_token([0.5] * 3, [], cfg(temperature=1.3, top_p=0.5), og.Rng(seed))
        assert got == (0 if u * 2 <= 1 else 1)
        # top_k 2 with a banned first id: ids 1 and 2 remain
        got = og.sample_token([0.5] * 3, [], cfg(temperature=1.3, top_k=2, top_p=1.0),
                              og.Rng(seed), [0])
        assert got == (1 if u * 2 <= 1 else 2)


def test_oracle_frequencies_follow_the_nucleus():
    logits = np.array([1.0, 0.5, 0.0, -1.0, 2.0])
    T, top_p, N = 0.7, 0.9, 20000
    p = np.exp((logits - logits.max()) / T)
    order = np.argsort(-p, kind="stable")
    cum, keep = 0.0, []
    for i in order:  # the smallest prefix whose mass reaches top_p of the total
        cum += p[i]
        keep.append(i)
        if cum >= top_p * p.sum():
            break
    q = np.zeros(5)
    q[keep] = p[keep] / p[keep].sum()
    rng = og.Rng(7)
    counts = np.zeros(5)
    c = cfg(temperature=T, top_p=top_p)
    for _ in range(N):
        counts[og.sample_token(logits, [], c, rng)] += 1
    f = counts / N
    for i in range(5):
        assert abs(f[i] - q[i]) <= 4 * math.sqrt(max(q[i] * (1 - q[i]), 1e-12) / N) + 1e-12
    assert counts[[i for i in range(5) if i not in keep]].sum() == 0


# ---------------------------------------------------- library vs oracle ----
def test_sampler_matches_oracle():
    import cpp_inference_train_engine_amd as mla
    rng = np.random.default_rng(11)
    for trial in range(300):
        V = int(rng.integers(2, 300))
        logits = (np.round(rng.normal(size=V) * 3, 1) if trial % 2 else
                  rng.normal(size=V) * 3).astype(np.float32)
        hist = rng.integers(0, V + 2, int(rng.integers(0, 12))).tolist()
        ban = rng.integers(0, V + 2, int(rng.integers(0, 6))).tolist()
        c = cfg(temperature=float(rng.choice([0.0, 0.3, 0.8, 1.5])),
                top_k=int(rng.choice([0, 1, 5, 40])), top_p=float(rng.choice([1.0, 0.95, 0.5])),
                repetition_penalty=float(rng.choice([1.0, 1.3, 0.7])),
                seed=int(rng.integers(0, 2**63)))
        state = int(rng.integers(0, 2**63))
        r = og.Rng(state)
        try:
            want = og.sample_token(logits, hist, c, r, ban)
        except og.SettingsError:
            with pytest.raises(mla.MlaError):
                mla.sample_token(logits, hist, gen_config(c), state, ban)
            continue
        got, new_state = mla.sample_token(logits, hist, gen_config(c), state, ban)
        assert (got, new_state) == (want, r.state), trial


def test_sampler_errors():
    import cpp_inference_train_engine_amd as mla
    G = mla.GenerationConfig
    cases = [
        (dict(logits=[1.0, float("nan")]), G(), "numerical_error", "Invalid sampler logits"),
        (dict(logits=[]), G(), "numerical_error", "Invalid sampler logits"),
        (dict(logits=[1.0, 2.0], banned=[0, 1]), G(temperature=0), "invalid_argument",
         "All tokens are banned"),
        (dict(logits=[1.0, 2.0], banned=[0, 1]), G(), "invalid_argument", "All tokens are banned"),
        (dict(logits=[1.0]), G(top_p=0), "invalid_argument", "Invalid generation settings"),
        (dict(logits=[1.0]), G(temperature=-1), "invalid_argument", "Invalid generation settings"),
        (dict(logits=[1.0]), G(repetition_penalty=0), "invalid_argument",
         "Invalid generation settings"),
        (dict(logits=[1.0]), G(max_new_tokens=65536), "invalid_argument",
         "Invalid generation settings"),
        (dict(logits=[1.0]), G(stop=("",)), "invalid_argument", "Stop strings must be nonempty"),
        (dict(logits=[1.0]), G(stop_tokens=((),)), "invalid_argument",
         "Stop token sequences must be nonempty"),
    ]
    for kw, c, code, msg in cases:
        with pytest.raises(mla.MlaError) as e:
            mla.sample_token(kw["logits"], [], c, None, kw.get("banned", ()))
        assert e.value.code == code and msg in str(e.value), (kw, c)


def test_banned_ids_of_the_reference_tokenizers():
    import cpp_inference_train_engine_amd as mla
    for name in ("tokenizer_tiny.json", "tokenizer_pilot.json"):
        t = mla.HipTokenizer(os.path.join(GOLDEN, name))
        with open(os.path.join(GOLDEN, name)) as f:
            merges = len(json.load(f)["merges"])
        V, eos = t.vocab_size, t.special("<|eos|>")
        want = [i for i in range(V) if (i >= V - 8 and i != eos) or 256 + merges <= i < V - 8]
        assert mla.banned_tokens(t) == want


# ------------------------------------------------------- the loop itself ----
class _Scripted:
    """An execution whose logits come from a seeded stream (one vector per call)."""

    def __init__(self, vocab, seed, max_sequence_length=64, peaks=None, ascii_only=False):
        self.vocab, self.rng = vocab, np.random.default_rng(seed)
        self.peaks = list(peaks) if peaks is not None else None
        self.max_sequence_length = max_sequence_length
        self.ascii_only = ascii_only
        self.calls = []

    def _logits(self):
        if self.peaks is not None:
            x = np.zeros(self.vocab, np.float32)
            x[self.peaks.pop(0)] = 1.0
            return x
        x = (self.rng.normal(size=self.vocab) * 2).astype(np.float32)
        if self.ascii_only:  # ids past 127 practically never drawn
            x[128:] -= 1000.0
        return x

    def prefill(self, ids):
        self.calls.append(("prefill", list(ids)))
        return self._logits()

    def decode(self, token):
        self.calls.append(("decode", int(token)))
        return self._logits()


def _token_bytes(t):
    return [t.decode([i]) if i not in set(_unassigned(t)) else b"" for i in range(t.vocab_size)]


def _unassigned(t):
    import cpp_inference_train_engine_amd as mla
    eos = t.special("<|eos|>")
    return [i for i in mla.banned_tokens(t) if i < t.vocab_size - 8 or i == eos]


def _ab_tokenizer(tmp_path):
    """The tiny tokenizer with merges a+b -> 256, 256+a -> 257 (vocab 266)."""
    with open(TOK_TINY) as f:
        j = json.load(f)
    j["vocab_size"] = 266
    j["merges"] = [[97, 98, 256], [256, 97, 257]]
    j["specials"] = {k: v + 2 for k, v in j["specials"].items()}
    path = str(tmp_path / "ab.json")
    with open(path, "w") as f:
        json.dump(j, f)
    return path


def _compare(t, c, prompt, seed, cancel_at=None):
    import cpp_inference_train_engine_amd as mla
    tb = _token_bytes(t)
    eos = t.special("<|eos|>")

    def make_cb(chunks):
        calls = [0]

        def cb(text):
            calls[0] += 1
            chunks.append(text.decode() if isinstance(text, bytes) else text)
            return cancel_at is None or calls[0] < cancel_at
        return cb

    want_chunks, got_chunks = [], []
    ex = _Scripted(t.vocab_size, seed)
    want = og.generate_tokens(ex.prefill, ex.decode, tb, eos, prompt, c, 64, make_cb(want_chunks))
    ex2 = _Scripted(t.vocab_size, seed)
    got = mla.generate_ids(ex2, t, prompt, gen_config(c), 64, make_cb(got_chunks))
    assert (got["tokens"], got["text"], got["finish_reason"]) == \
        (want["tokens"], want["text"], want["finish_reason"])
    assert got_chunks == want_chunks
    assert ex2.calls == ex.calls  # same prefill and decodes, none after the last token
    return got


def test_generation_matches_oracle(tmp_path):
    import cpp_inference_train_engine_amd as mla
    rng = np.random.default_rng(5)
    for path in (TOK_TINY, _ab_tokenizer(tmp_path)):
        t = mla.HipTokenizer(path)
        letters = [b"a", b"b", b"ab", b"ba", b"\n", b"a\xc3", b"\xc3\xa9"]
        for trial in range(60):
            stop = tuple(letters[i] for i in rng.choice(len(letters), int(rng.integers(0, 3)),
                                                        replace=False))
            seqs = tuple(tuple(int(x) for x in rng.integers(0, 258, int(rng.integers(1, 3))))
                         for _ in range(int(rng.integers(0, 3))))
            c = cfg(max_new_tokens=int(rng.integers(0, 24)),
                    temperature=float(rng.choice([0.0, 0.0, 0.7, 1.5])),
                    top_k=int(rng.choice([0, 3])), top_p=float(rng.choice([1.0, 0.9])),
                    repetition_penalty=float(rng.choice([1.0, 1.2])),
                    seed=int(rng.integers(0, 2**32)), stop=stop, stop_tokens=seqs)
            prompt = [t.special("<|bos|>")] + rng.integers(0, 256, int(rng.integers(1, 8))).tolist()
            _compare(t, c, prompt, seed=trial,
                     cancel_at=int(rng.integers(1, 6)) if trial % 7 == 3 else None)


def test_generation_stop_rules():
    """generate_tokens' stop rules (inference.cpp:504-560) on scripted argmaxes: EOS ends
    without text, a stop token sequence ends with its text removed, the first listed
    stop string that occurs cuts the text; the last token is never decoded; banned ids
    (specials other than EOS) are skipped."""
    import cpp_inference_train_engine_amd as mla
    t = mla.HipTokenizer(TOK_TINY)
    eos, bos = t.special("<|eos|>"), t.special("<|bos|>")
    G = mla.GenerationConfig
    ex = _Scripted(264, 0, peaks=[72, 105, eos, 0])
    out = mla.generate(ex, t, "Q", G(max_new_tokens=8, temperature=0))
    assert out["tokens"] == [72, 105, eos] and out["text"] == "Hi" and \
        out["finish_reason"] == "stop"
    assert ex.calls == [("prefill", [bos, 81]), ("decode", 72), ("decode", 105)]
    ex = _Scripted(264, 0, peaks=[65, 66, 67, 68])
    out = mla.generate(ex, t, "Q", G(max_new_tokens=8, temperature=0, stop_tokens=((66, 67),)))
    assert out["tokens"] == [65, 66, 67] and out["text"] == "A"
    ex = _Scripted(264, 0, peaks=[65, 66, 67, 68, 69])
    out = mla.generate(ex, t, "Q", G(max_new_tokens=8, temperature=0, stop=("CD", "B")))
    assert out["text"] == "A" and out["finish_reason"] == "stop"
    ex = _Scripted(264, 0, peaks=[65, 66, 67])
    out = mla.generate(ex, t, "Q", G(max_new_tokens=3, temperature=0))
    assert out["finish_reason"] == "length" and len(ex.calls) == 3  # prefill + 2 decodes
    ex = _Scripted(264, 0, peaks=[bos, 70])  # the peak is banned: the next best (id 0) wins
    out = mla.generate(ex, t, "Q", G(max_new_tokens=1, temperature=0))
    assert out["tokens"] == [0]
    with pytest.raises(mla.MlaError):
        mla.generate(_Scripted(264, 0, peaks=[1]), t, "Q" * 60, G(max_new_tokens=8))
    with pytest.raises(mla.MlaError):
        mla.generate(_Scripted(264, 0, peaks=[1]), t, "Q", G(max_new_tokens=4,
                                                              stop_tokens=((300,),)))


def test_streamed_text_is_the_text(tmp_path):
    """Chunks handed to the callback add up to the final text (the reference's HTTP test
    compares the streamed and the plain completion, tests/test_tools.py:672-683) when
    stop strings hold text back (ASCII text: with invalid bytes the chunks are cleaned
    one by one, as the reference cleans them)."""
    import cpp_inference_train_engine_amd as mla
    t = mla.HipTokenizer(_ab_tokenizer(tmp_path))
    for seed in range(40):
        chunks = []
        out = mla.generate_ids(_Scripted(t.vocab_size, seed, ascii_only=True), t,
                               [t.special("<|bos|>"), 97],
                               gen_config(cfg(max_new_tokens=20, stop=("ba",), seed=seed)), 64,
                               lambda s: chunks.append(s) or True)
        assert "".join(chunks) == out["text"]
