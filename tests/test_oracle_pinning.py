"""Pins the CPU oracle (oracle/mla_oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the restatement fails it:
golden vectors held by the reference, the reference's own Rng built from its
header, closed forms, invariants, and brute force on tiny inputs.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN, MLA36M, TINY


# ------------------------------------------------------------ golden data ----
def test_forward_matches_reference_fixture(orc, tiny_fixture):
    """docs/verification/attention-sync/oracle: weights + ids -> engine logits [9x264].
    PyTorch agreed with these logits to 2.15e-6 (flash-oracle-report.json)."""
    cfg = orc.Config.from_dict(tiny_fixture["config"])
    assert orc.parameter_count(cfg) == tiny_fixture["parameter_count"] == 26704
    logits = orc.forward(cfg, tiny_fixture["params"], tiny_fixture["tokens"])
    assert logits.shape == (9, 264)
    np.testing.assert_allclose(logits, tiny_fixture["logits"], rtol=0, atol=1e-5)


def test_forward_fixture_catches_planted_mistakes(orc, tiny_fixture):
    """The fixture is sensitive: perturbing one weight of a late layer moves the logits."""
    cfg = orc.Config.from_dict(tiny_fixture["config"])
    p = tiny_fixture["params"].copy()
    p[-1] += 0.05  # last element of layers.1.ffn.w_down
    logits = orc.forward(cfg, p, tiny_fixture["tokens"])
    assert np.abs(logits - tiny_fixture["logits"]).max() > 1e-4


def test_rng_matches_reference_rng_vectors(orc):
    """Known answers from the reference's include/mini_mla/rng.hpp (oracle/_ref)."""
    vec = json.load(open(os.path.join(GOLDEN, "rng_vectors.json")))
    for key, values in vec.items():
        kind, seed, bound = key.split("/")
        r = orc.Rng(int(seed))
        for want in values:
            if kind == "next":
                assert r.next() == int(want)
            elif kind == "uniform":
                assert np.float32(r.uniform()) == np.float32(float(want))
            elif kind == "normal":
                assert np.float32(r.normal()) == np.float32(float(want))
            else:
                assert r.bounded(int(bound)) == int(want)


def test_rng_live_reference_build_when_present(orc):
    """Re-runs the reference Rng (oracle/_ref/rng_ref) when it was built here."""
    got = orc.ref_rng("normal", 1234, 200)
    if got is None:
        pytest.skip("oracle/_ref not built (no reference checkout)")
    r = orc.Rng(1234)
    assert [np.float32(r.normal()) for _ in range(200)] == [np.float32(float(x)) for x in got]


def test_splitmix64_closed_form(orc):
    """Textbook SplitMix64 first outputs for seed 0."""
    r = orc.Rng(0)
    assert r.next() == 0xE220A8397B1DCDAF
    assert r.next() == 0x6E789E6AA1B965F4


# ---------------------------------------------------------------- config ----
def test_parameter_count_known_answers(orc):
    """tests/test_model.cpp:21-28: mla36m has 35,763,840 parameters."""
    assert orc.parameter_count(orc.Config.from_dict(MLA36M)) == 35763840
    assert orc.parameter_count(orc.Config.from_dict(TINY)) == 26704
    shapes = orc.parameter_shapes(orc.Config.from_dict(MLA36M))
    assert sum(r * c for r, c in shapes) == 35763840
    assert shapes[0] == (16384, 512) and shapes[2 + 8] == (512, 512)  # w_o = [H*dv x d]


def test_config_validation_rejects_bad_shapes(orc):
    """config.cpp:20-48: odd RoPE width, indivisible d_model, bad theta rejected."""
    assert orc.validate(orc.Config.from_dict(MLA36M))
    for key, value in [("head_dim_rope", 15), ("d_model", 500), ("rope_theta", 1.0),
                       ("n_layers", 0), ("vocab_size", 70000), ("norm_epsilon", 0.0)]:
        bad = dict(MLA36M, **{key: value})
        assert not orc.validate(orc.Config.from_dict(bad)), key


def test_model_init_registry_order(orc):
    """model.cpp:20-75: norms are 1, matrices N(0,0.02) drawn in registry order,
    residual matrices (w_o, w_down) scaled by 1/sqrt(2L)."""
    cfg = orc.Config.from_dict(TINY)
    p = orc.model_init(cfg, 7)
    r = orc.Rng(7)
    first = np.array([r.normal() * np.float32(0.02) for _ in range(8)], np.float32)
    np.testing.assert_array_equal(p[:8], first)
    shapes = orc.parameter_shapes(cfg)
    offs = np.cumsum([0] + [a * b for a, b in shapes])
    assert np.all(p[offs[1]:offs[2]] == 1.0)  # final_norm
    w_o = p[offs[2 + 8]:offs[2 + 9]]
    w_dq = p[offs[2 + 1]:offs[2 + 2]]
    assert 0.4 < w_o.std() / w_dq.std() < 0.6  # 1/sqrt(2L) = 0.5


# ----------------------------------------------------------- 16-bit casts ----
def test_f16_rounding_is_ieee_rne(orc):
    """io.cpp:152-158 to_half == static_cast<_Float16>: compare with numpy's RNE cast
    on every fp16 boundary pattern plus random values, subnormals, overflow, NaN."""
    rng = np.random.default_rng(0)
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    exact = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(exact)
    vals = [exact[finite]]
    # midpoints between consecutive halves and their neighbours (ties to even)
    nxt = np.nextafter(exact[finite].astype(np.float16), np.float16(np.inf)).astype(np.float32)
    mid = ((exact[finite].astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)
    vals += [mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(-np.inf))]
    vals += [rng.standard_normal(200000).astype(np.float32) * s for s in (1e-6, 1e-3, 1, 1e3, 7e4)]
    vals += [np.array([65504, 65519.99, 65520, 1e9, -65520, 2.0 ** -25, 2.0 ** -24, 0.0, -0.0],
                      np.float32)]
    x = np.concatenate(vals)
    x = x[np.isfinite(x)]
    got = orc.round_f16(x)
    want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)
    assert orc.round_f16(np.array([np.nan], np.float32))[0] & 0x7e00 == 0x7e00


def test_bf16_rounding_is_rne(orc):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32),
                        (rng.integers(0, 1 << 32, 100000, dtype=np.uint64).astype(np.uint32))
                        .view(np.float32)])
    x = x[np.isfinite(x)]
    got = orc.round_bf16(x).astype(np.uint32)
    u = x.view(np.uint32).astype(np.uint64)
    want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) & 0xFFFF
    np.testing.assert_array_equal(got, want)
    # brute-force definition: nearest of the two bracketing bf16 values, ties to even
    s = x[np.abs(x) < 1e38][:5000]
    hi = (s.view(np.uint32) >> 16).astype(np.uint32)
    c0 = (hi << 16).view(np.float32).astype(np.float64)
    c1 = ((hi + 1) << 16).view(np.float32).astype(np.float64)
    d0, d1 = np.abs(s - c0), np.abs(c1 - s)
    pick = np.where((d0 < d1) | ((d0 == d1) & (hi % 2 == 0)), c0, c1)
    got64 = orc.bits_to_f32(orc.round_bf16(s), 1).astype(np.float64)
    np.testing.assert_array_equal(got64, pick)


# --------------------------------------------------------------- decode ----
SMALL = dict(vocab_size=64, max_sequence_length=32, n_layers=2, d_model=32, n_heads=2,
             head_dim_nope=8, head_dim_rope=4, head_dim_value=8, q_lora_rank=16,
             kv_lora_rank=8, d_ff=48, norm_epsilon=1e-5, rope_theta=10000.0)


@pytest.mark.parametrize("absorbed", [True, False])
def test_decode_matches_full_recomputation(orc, absorbed):
    """test_training.cpp:52-76: cached decode logits == forward row, |d| < 2e-5, 20 steps,
    for the absorbed and the reconstructed-K/V attention."""
    cfg = orc.Config.from_dict(SMALL)
    params = orc.model_init(cfg, 21)
    dec = orc.Decoder(cfg, params, absorbed=absorbed)
    ids = [1, 2, 3]
    dec.prefill(ids)
    for i in range(20):
        tok = i % 16
        ids.append(tok)
        got = dec.decode(tok)
        want = orc.forward(cfg, params, ids)[-1]
        assert np.abs(got - want).max() < 2e-5


def test_decode_rejects_invalid_position_and_token(orc):
    """inference.cpp:71-75."""
    cfg = orc.Config.from_dict(SMALL)
    params = orc.model_init(cfg, 3)
    dec = orc.Decoder(cfg, params)
    with pytest.raises(ValueError):
        dec.decode(1)  # no prefill
    dec.prefill([1, 2])
    with pytest.raises(ValueError):
        dec.decode(cfg.vocab_size)
    dec.prefill(list(range(31)))
    dec.decode(1)  # position 31 is the last slot
    with pytest.raises(ValueError):
        dec.decode(1)


def test_decode_on_fixture_weights_matches_fixture_logits(orc, tiny_fixture):
    """Decode of ids[1:] after prefilling ids[:1] reproduces every fixture logit row."""
    cfg = orc.Config.from_dict(tiny_fixture["config"])
    dec = orc.Decoder(cfg, tiny_fixture["params"])
    toks = tiny_fixture["tokens"].tolist()
    rows = [dec.prefill(toks[:1])] + [dec.decode(t) for t in toks[1:]]
    np.testing.assert_allclose(np.stack(rows), tiny_fixture["logits"], atol=2e-5, rtol=0)


# ---------------------------------------------------- paged attention ----
def _paged_case(rng, B, H, kv, rp, ps, dtype, q_lens=None, max_len=300):
    lens = rng.integers(1, max_len, B).astype(np.int32)
    q_lens = np.ones(B, np.int32) if q_lens is None else np.asarray(q_lens, np.int32)
    lens = np.maximum(lens, q_lens)
    need = (lens + ps - 1) // ps
    max_pages = int(need.max())
    P = int(need.sum()) + 3
    perm = rng.permutation(P).astype(np.int32)
    table = np.full((B, max_pages), -1, np.int32)
    o = 0
    for b in range(B):
        table[b, :need[b]] = perm[o:o + need[b]]
        o += need[b]
    vals = rng.standard_normal((P, ps * (kv + rp))).astype(np.float32)
    bits = (orc_round(vals, dtype))
    rows = int(q_lens.sum())
    ql = rng.standard_normal((rows, H, kv)).astype(np.float32)
    qr = rng.standard_normal((rows, H, rp)).astype(np.float32)
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    return lens, table, bits, ql, qr, cu_q


def orc_round(x, dtype):
    import oracle
    return oracle.round_f16(x) if dtype == 0 else oracle.round_bf16(x)


def _words(sl, kv, rp, ps):
    """Independent statement of the page-record format: row-major, or MFMA-tiled
    (16-token tiles x 32-column K-steps x 8-column groups) when ps%16, kv%32, rp%8 == 0."""
    r = np.arange(kv)[None, :]
    c = np.arange(rp)[None, :]
    s = sl[:, None]
    if ps % 16 or kv % 32 or rp % 8:
        return s * kv + r, ps * kv + s * rp + c
    lat = (((s // 16) * (kv // 32) + r // 32) * 4 + (r % 32) // 8) * 128 + (s % 16) * 8 + r % 8
    rope = ps * kv + ((s // 16) * (rp // 8) + c // 8) * 128 + (s % 16) * 8 + c % 8
    return lat, rope


def _brute(lens, table, bits, ql, qr, cu_q, H, kv, rp, ps, dtype, scale):
    import oracle
    vals = oracle.bits_to_f32(bits, dtype).astype(np.float64)
    out = np.zeros(ql.shape, np.float64)
    for b in range(len(lens)):
        nq = cu_q[b + 1] - cu_q[b]
        toks = np.arange(lens[b])
        pg = table[b, toks // ps]
        sl = toks % ps
        lw, rw = _words(sl, kv, rp, ps)
        C = vals[pg[:, None], lw]
        K = vals[pg[:, None], rw]
        for i in range(nq):
            row = cu_q[b] + i
            L = lens[b] - nq + i + 1
            for h in range(H):
                s = (C[:L] @ ql[row, h].astype(np.float64) + K[:L] @ qr[row, h]) * scale
                p = np.exp(s - s.max())
                out[row, h] = p @ C[:L] / p.sum()
    return out


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("shape", [(3, 16, 4, 8), (2, 32, 8, 16)], ids=["rowmajor", "tiled"])
def test_attention_paged_brute_force_fp64(orc, dtype, shape):
    """Closed form: softmax-weighted latent sum, in fp64 numpy over the same 16-bit data,
    including causal rows of a prefill chunk (q_len > 1); both page-record formats."""
    rng = np.random.default_rng(5 + dtype)
    H, kv, rp, ps = shape
    lens, table, bits, ql, qr, cu_q = _paged_case(rng, 5, H, kv, rp, ps, dtype,
                                                   q_lens=[1, 4, 1, 2, 1], max_len=60)
    scale = 1.0 / np.sqrt(12.0)
    got = orc.attention_paged(H, kv, rp, ps, dtype, cu_q, lens, table, bits, ql, qr, scale)
    want = _brute(lens, table, bits, ql, qr, cu_q, H, kv, rp, ps, dtype, scale)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_attention_paged_equals_contiguous_decoder_cache(orc):
    """Permuting pages changes nothing: same output as an identity page table."""
    rng = np.random.default_rng(9)
    H, kv, rp, ps = 2, 8, 4, 4
    lens, table, bits, ql, qr, cu_q = _paged_case(rng, 4, H, kv, rp, ps, 0, max_len=40)
    scale = 0.25
    got = orc.attention_paged(H, kv, rp, ps, 0, cu_q, lens, table, bits, ql, qr, scale)
    # gather into contiguous pages 0..n-1
    rec = ps * (kv + rp)
    flat = []
    table2 = np.full_like(table, -1)
    k = 0
    for b in range(len(lens)):
        for j in range((lens[b] + ps - 1) // ps):
            flat.append(bits[table[b, j]])
            table2[b, j] = k
            k += 1
    got2 = orc.attention_paged(H, kv, rp, ps, 0, cu_q, lens, table2, np.stack(flat), ql, qr, scale)
    np.testing.assert_array_equal(got, got2)
    assert bits.shape[1] == rec


def test_attention_paged_threads_change_no_bit(orc):
    """The CPU baseline runs sessions on several threads; every result bit must equal the
    one-thread run (sessions are independent)."""
    rng = np.random.default_rng(13)
    H, kv, rp, ps = 4, 32, 8, 16
    lens, table, bits, ql, qr, cu_q = _paged_case(rng, 9, H, kv, rp, ps, 0, max_len=90)
    one = orc.attention_paged(H, kv, rp, ps, 0, cu_q, lens, table, bits, ql, qr, 0.3,
                              want_lse=True, threads=1)
    many = orc.attention_paged(H, kv, rp, ps, 0, cu_q, lens, table, bits, ql, qr, 0.3,
                               want_lse=True, threads=4)
    np.testing.assert_array_equal(one[0], many[0])
    np.testing.assert_array_equal(one[1], many[1])


def test_attention_lse(orc):
    rng = np.random.default_rng(2)
    H, kv, rp, ps = 2, 8, 4, 4
    lens, table, bits, ql, qr, cu_q = _paged_case(rng, 3, H, kv, rp, ps, 0, max_len=20)
    out, lse = orc.attention_paged(H, kv, rp, ps, 0, cu_q, lens, table, bits, ql, qr, 0.5,
                                   want_lse=True)
    vals = orc.bits_to_f32(bits, 0).astype(np.float64)
    b, h = 1, 1
    toks = np.arange(lens[b])
    C = vals[table[b, toks // ps][:, None], (toks % ps)[:, None] * kv + np.arange(kv)]
    K = vals[table[b, toks // ps][:, None], ps * kv + (toks % ps)[:, None] * rp + np.arange(rp)]
    s = (C @ ql[b, h] + K @ qr[b, h]) * 0.5
    assert abs(lse[b, h] - np.log(np.exp(s).sum())) < 1e-4


# ---------------------------------------------------------------- greedy ----
def test_greedy_sampler_semantics(orc):
    """test_training.cpp:77-110 greedy part: argmax, repetition penalty, banned, ties."""
    scores = np.array([2, -1, 1, 0], np.float32)
    assert orc.greedy(scores) == 0
    assert orc.greedy(scores, history=[0, 0], repetition_penalty=3) == 2
    assert orc.greedy(scores, banned=[0, 1, 2, 3]) == -1
    assert orc.greedy(np.array([1, 3, 3, 0], np.float32)) == 1  # lowest index on ties
    assert orc.greedy(np.array([-2, -1], np.float32), history=[1], repetition_penalty=4) == 0
    assert orc.greedy(np.array([0, np.inf], np.float32)) == -2


@pytest.mark.parametrize("shape", [(8, 4, 16), (128, 16, 64), (32, 8, 16)])
def test_append_places_every_value_at_its_layout_word(orc, shape):
    """orc_append_paged writes column r of token slot s to the record word that the
    independent format statement (_words) names, and nowhere else."""
    kv, rp, ps = shape
    rng = np.random.default_rng(4)
    P, T = 3, 2 * ps
    slots = rng.permutation(P * ps)[:T].astype(np.int32)
    ckv = (np.arange(T * kv, dtype=np.float32).reshape(T, kv) % 2000) + 1
    kr = -((np.arange(T * rp, dtype=np.float32).reshape(T, rp) % 2000) + 1)
    pages = np.zeros((P, ps * (kv + rp)), np.uint16)
    orc.append_paged(kv, rp, ps, 0, ckv, kr, slots, pages)
    vals = orc.bits_to_f32(pages, 0)
    seen = np.zeros(pages.shape, bool)
    for t in range(T):
        pg, sl = slots[t] // ps, slots[t] % ps
        lw, rw = _words(np.array([sl]), kv, rp, ps)
        np.testing.assert_array_equal(vals[pg, lw[0]], ckv[t])
        np.testing.assert_array_equal(vals[pg, rw[0]], kr[t])
        seen[pg, lw[0]] = True
        seen[pg, rw[0]] = True
    assert np.all(vals[~seen] == 0)


def test_blas_path_equals_the_loops(orc):
    """The CPU baseline times the oracle with its products on a portable CBLAS (numpy's
    OpenBLAS, standing in for the reference's Accelerate calls); that path must compute
    what the pinned loops compute, up to summation order: the full forward and absorbed
    decode agree within 1e-5 of the logits' scale on a small random model."""
    from conftest import MLA36M
    cfgd = dict(MLA36M, n_layers=2, vocab_size=2048, max_sequence_length=128)
    cfg = orc.Config.from_dict(cfgd)
    params = orc.model_init(cfg, 5)
    ids = orc.Rng(5).bounded_many(cfg.vocab_size, 48).astype(np.uint16)

    def run():
        d = orc.Decoder(cfg, params, absorbed=True)
        pre = d.prefill(ids[:40])
        dec = [d.decode(int(t)) for t in ids[40:]]
        return pre, np.stack(dec), orc.forward(cfg, params, ids)

    loops = run()
    desc = orc.use_blas(True)
    try:
        if desc is None:
            pytest.skip("numpy ships no OpenBLAS here")
        blas = run()
    finally:
        orc.use_blas(False)
    for a, b in zip(loops, blas):
        scale = float(np.abs(a).max())
        assert np.abs(a - b).max() <= 1e-5 * max(scale, 1.0)
    assert "OpenBLAS" in desc
