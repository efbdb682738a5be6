"""Tokenizer (mla_tokenizer_*, HipTokenizer) and text generation against the reference.

Known answers from the reference's own tests (tests/test_files.cpp:68-107) on its own
tokenizer files (tests/golden/tokenizer_tiny.json = examples/tokenizer.json,
tests/golden/tokenizer_pilot.json = examples/pilot-tokenizer.json): raw bytes and
special tokens round-trip, ``encode("ababa") == [256, 257]`` under merges
(a,b)->256, (256,a)->257, a merge naming a later id is refused.  Beyond those, the ranked
BPE is checked against a brute-force encoder written from the format's rule
(docs/file_formats.md: "Ranked merges are applied with stable left-position tie
breaking"): repeatedly merge the lowest-id pair, leftmost first.  Host code: CPU tests;
generation with this tokenizer is tested in test_generation.py and test_serving.py.
"""
import hashlib
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN, TINY

TOK_TINY = os.path.join(GOLDEN, "tokenizer_tiny.json")
TOK_PILOT = os.path.join(GOLDEN, "tokenizer_pilot.json")


def _tok(path):
    import cpp_inference_train_engine_amd as mla
    return mla.HipTokenizer(path)


def _write(tmp_path, obj, name="tokenizer.json"):
    path = str(tmp_path / name)
    with open(path, "w") as f:
        json.dump(obj, f)
    return path


def _brute_force(merges, data: bytes):
    """Lowest merged id first, leftmost first: one merge per pass over the sequence."""
    rank = {(l, r): i for l, r, i in merges}
    seq = list(data)
    while True:
        best = None
        for k in range(len(seq) - 1):
            i = rank.get((seq[k], seq[k + 1]))
            if i is not None and (best is None or i < best[0]):
                best = (i, k)
        if best is None:
            return seq
        i, k = best
        seq[k:k + 2] = [i]


# ------------------------------------------------------- known answers ----
def test_reference_files_and_hashes():
    for path in (TOK_TINY, TOK_PILOT):
        t = _tok(path)
        with open(path, "rb") as f:
            raw = f.read()
        assert t.hash == hashlib.sha256(raw).hexdigest()
        assert t.vocab_size == json.loads(raw)["vocab_size"]
        assert [t.special(n) for n in ("<|pad|>", "<|bos|>", "<|eos|>")] == \
            [t.vocab_size - 8, t.vocab_size - 7, t.vocab_size - 6]


def test_raw_bytes_and_specials_are_unambiguous():
    """test_files.cpp:68-86."""
    t = _tok(TOK_TINY)
    text = "Hello, café 世界 🚀\n<|eos|>".encode() + b"\0"
    ids = t.encode(text)
    assert ids.tolist() == list(text)  # no merges: one id per byte, the spelling included
    assert t.decode(ids) == text
    assert t.encode("<|eos|>", allow_special=True).tolist() == [t.special("<|eos|>")]
    assert t.encode("a<|user|>b<|sep|>", allow_special=True).tolist() == \
        [97, t.special("<|user|>"), 98, t.special("<|sep|>")]


def _ab_tokenizer(merges):
    with open(TOK_TINY) as f:
        j = json.load(f)
    j["vocab_size"] = 266
    j["merges"] = merges
    j["specials"] = {k: v + 2 for k, v in j["specials"].items()}
    return j


def test_bpe_merge_priority(tmp_path):
    """test_files.cpp:87-107: encode("ababa") == [256, 257]."""
    t = _tok(_write(tmp_path, _ab_tokenizer([[97, 98, 256], [256, 97, 257]])))
    assert t.encode("ababa").tolist() == [256, 257]
    assert t.decode([256, 257]) == b"ababa"


def test_merge_naming_a_later_id_is_refused(tmp_path):
    import cpp_inference_train_engine_amd as mla
    with pytest.raises(mla.MlaError) as e:
        _tok(_write(tmp_path, _ab_tokenizer([[257, 98, 256]])))
    assert e.value.code == "invalid_argument"
    assert "BPE merge references a future token" in str(e.value)


# ------------------------------------------------------------ the BPE ----
def test_pilot_tokenizer_matches_brute_force():
    """The pilot tokenizer's 72 merges: random strings built from merge spellings and
    random bytes encode as the brute-force rule does, and decode back."""
    with open(TOK_PILOT) as f:
        merges = json.load(f)["merges"]
    t = _tok(TOK_PILOT)
    spell = {i: bytes([i]) for i in range(256)}
    for l, r, i in merges:
        spell[i] = spell[l] + spell[r]
    pieces = [spell[i] for _, _, i in merges]
    rng = np.random.default_rng(0)
    for trial in range(300):
        parts = []
        for _ in range(int(rng.integers(1, 40))):
            if rng.random() < 0.7:
                parts.append(pieces[int(rng.integers(len(pieces)))])
            else:
                parts.append(bytes(rng.integers(0, 256, int(rng.integers(1, 4)), dtype=np.uint8)))
        data = b"".join(parts)
        got = t.encode(data).tolist()
        assert got == _brute_force(merges, data), (trial, data)
        assert t.decode(got) == data


def test_overlapping_runs_resolve_leftmost(tmp_path):
    """With (a,a)->256 and (256,256)->257: 'aaa' -> [256, a], 'aaaa' -> [256, 256] -> [257],
    'aaaaa' -> [257, a] (leftmost pairs merge first)."""
    j = _ab_tokenizer([[97, 97, 256], [256, 256, 257]])
    t = _tok(_write(tmp_path, j))
    assert t.encode("aaa").tolist() == [256, 97]
    assert t.encode("aaaa").tolist() == [257]
    assert t.encode("aaaaa").tolist() == [257, 97]
    for n in range(12):
        assert t.encode(b"a" * n).tolist() == _brute_force(j["merges"], b"a" * n)


# ------------------------------------------------------------ errors ----
@pytest.mark.parametrize("edit,code,message", [
    (lambda j: j.update(format="other"), "unsupported", "Unsupported tokenizer format"),
    (lambda j: j.update(pretokenizer="regex"), "unsupported", "Unsupported tokenizer format"),
    (lambda j: j.update(vocab_size=100), "invalid_argument",
     "Tokenizer vocabulary must be in [264,65535]"),
    (lambda j: j.update(merges=[[97, 98, 300]]), "invalid_argument", "Malformed BPE merge"),
    (lambda j: j.update(merges=[[97, 98, 256], [97, 98, 257]]), "invalid_argument",
     "Duplicate BPE pair"),
    (lambda j: j["specials"].pop("<|sep|>"), "invalid_argument",
     "Tokenizer must define exactly eight special tokens"),
    (lambda j: j["specials"].update({"<|user|>": 257}), "invalid_argument",
     "Special token IDs disagree with the native chat template"),
])
def test_invalid_tokenizers(tmp_path, edit, code, message):
    import cpp_inference_train_engine_amd as mla
    j = _ab_tokenizer([])  # vocab 266: room for two merges
    _tok(_write(tmp_path, j, "ok.json"))
    edit(j)
    with pytest.raises(mla.MlaError) as e:
        _tok(_write(tmp_path, j))
    assert e.value.code == code and message in str(e.value)


def test_decode_rejects_unknown_ids_and_skips_specials():
    import cpp_inference_train_engine_amd as mla
    t = _tok(TOK_PILOT)
    unassigned = 256 + 72  # merge capacity without bytes (docs/file_formats.md)
    for bad in (unassigned, t.vocab_size):
        with pytest.raises(mla.MlaError) as e:
            t.decode([65, bad])
        assert e.value.code == "invalid_argument" and "Unknown token ID" in str(e.value)
    ids = [t.special("<|bos|>"), 72, 105, t.special("<|eos|>")]
    assert t.decode(ids) == b"<|bos|>Hi<|eos|>"
    assert t.decode(ids, skip_special=True) == b"Hi"


def test_chat_prompt_layout():
    """Tokenizer::chat_prompt (tokenizer.cpp:236-262)."""
    import cpp_inference_train_engine_amd as mla
    t = _tok(TOK_TINY)
    ids = t.chat_prompt([{"role": "system", "content": "S"}, {"role": "user", "content": "Hi"}])
    assert ids == [257, 261, 10, 83, 258, 10, 259, 10, 72, 105, 258, 10, 260, 10]
    with pytest.raises(mla.MlaError):
        t.chat_prompt([])
    with pytest.raises(mla.MlaError):
        t.chat_prompt([{"role": "robot", "content": "x"}])


def test_clean_utf8():
    """clean_utf8 (tokenizer.cpp:44-57): one U+FFFD per byte that starts no valid sequence."""
    from cpp_inference_train_engine_amd import clean_utf8
    assert clean_utf8("café 🚀".encode()) == "café 🚀"
    assert clean_utf8(b"a\xffb") == "a�b"
    assert clean_utf8(b"\xe2\x82") == "��"       # truncated 3-byte sequence
    assert clean_utf8(b"\xed\xa0\x80") == "�" * 3     # encoded surrogate
    assert clean_utf8(b"\xc0\x80") == "��"       # overlong NUL
