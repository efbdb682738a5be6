"""Session engine (mla_engine_* / mla_session_*): the reference's Execution contract.

Parity targets (reference tests in brackets):
  * prefill / decode logits against the oracle's CpuDecoder restatement on the same
    fp16-rounded weights (tests/test_mps.cpp:126-166 compares the MPS fp16 decode with
    the CPU path at 0.015; here LOGIT_ATOL);
  * cached decode equals full recomputation (tests/test_training.cpp:52-76), on the GPU:
    prefill(prompt) + decode(t_1..t_k) against prefill(prompt + t_1..t_k);
  * forked sessions decoding concurrently on threads equal serial runs
    (tests/inference_sessions.hpp:10-58, 191-217);
  * invalid position / token / prompt rejected with invalid_argument
    (src/infer/inference.cpp:48-50,71-75).
Config 1 (tiny-test, Model::create seed 0, 32-token prompt, 32 greedy steps) runs on the
oracle (CPU) and through the engine (GPU).
"""
import sys
import threading

import numpy as np
import pytest

from conftest import MLA36M, TINY

LOGIT_ATOL = 5e-3


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _models(cfgd, seed=0):
    import oracle
    ocfg = oracle.Config.from_dict(cfgd)
    params = oracle.model_init(ocfg, seed)
    p16 = oracle.bits_to_f32(oracle.round_f16(params))
    return ocfg, params, p16


def _prompt(n, vocab, seed=0):
    import oracle
    return oracle.Rng(seed).bounded_many(vocab, n).astype(np.uint16)


def _engine(mla, cfgd, params, **kw):
    return mla.HipEngine(mla.ModelConfig.from_dict(cfgd), params, **kw)


def _margin_ok(logits):
    top2 = np.sort(logits)[-2:]
    return top2[1] - top2[0] > 2 * LOGIT_ATOL


# ------------------------------------------------------------------ CPU ----
def test_config1_generation_on_the_oracle(orc):
    """Config 1 on the reference CPU path (restated): prefill 32 random ids, 32 greedy
    steps; every decode's logits equal the full forward's row (2e-5, test_training.cpp:
    52-76) and the greedy tokens are the forward's argmaxes."""
    cfg, params, _ = _models(TINY)
    prompt = _prompt(32, TINY["vocab_size"])
    dec = orc.Decoder(cfg, params)
    logits = dec.prefill(prompt)
    seq = list(prompt)
    for i in range(32):
        tok = int(np.argmax(logits))
        seq.append(tok)
        if i + 1 < 32:
            logits = dec.decode(tok)
            full = orc.forward(cfg, params, seq)[-1]
            np.testing.assert_allclose(logits, full, atol=2e-5, rtol=0)
    assert len(seq) == 64 and max(seq) < TINY["vocab_size"]


# ------------------------------------------------------------------ GPU ----
@pytest.mark.gpu
def test_config1_tiny_engine_matches_oracle(gpu, orc):
    """tiny-test through the engine: prefill, 32 teacher-forced decode steps and the free
    greedy generation, against the oracle on the same fp16 weights."""
    cfg, params, p16 = _models(TINY)
    prompt = _prompt(32, TINY["vocab_size"])
    eng = _engine(gpu, TINY, params, max_sessions=2, max_rows=64, num_pages=16, page_size=16)
    ex = eng.session()
    dec = orc.Decoder(cfg, p16, round_cache=True)
    got, want = ex.prefill(prompt), dec.prefill(prompt)
    assert np.abs(got - want).max() <= LOGIT_ATOL
    for i in range(31):
        tok = int(np.argmax(want))
        got, want = ex.decode(tok), dec.decode(tok)
        err = np.abs(got - want).max()
        assert err <= LOGIT_ATOL, f"step {i}: {err}"
    assert ex.position == 63
    # free-running greedy generation (generate_tokens, inference.cpp:469-579)
    ex2, dec2 = eng.session(), orc.Decoder(cfg, p16, round_cache=True)
    toks = gpu.generate_tokens(ex2, prompt, 32, TINY["max_sequence_length"])
    logits = dec2.prefill(prompt)
    for i, t in enumerate(toks):
        if not _margin_ok(logits):
            break  # a near tie may legitimately flip; the sequences may diverge from here
        assert t == int(np.argmax(logits)), f"token {i}"
        logits = dec2.decode(t)
    _say(f"config1 tokens: {toks}")
    eng.close()


@pytest.mark.gpu
def test_mla36m_engine_matches_oracle(gpu, orc):
    """mla36m: a 100-token prompt prefilled in chunks of 48 (chunked prefill on top of the
    session's own context), then 6 decode steps, against the oracle."""
    cfg, params, p16 = _models(MLA36M)
    prompt = _prompt(100, MLA36M["vocab_size"], seed=1)
    eng = _engine(gpu, MLA36M, params, max_sessions=2, max_rows=48, num_pages=8)
    ex = eng.session()
    dec = orc.Decoder(cfg, p16, round_cache=True)
    got, want = ex.prefill(prompt), dec.prefill(prompt)
    _say(f"prefill max err {np.abs(got - want).max():.3e}")
    assert np.abs(got - want).max() <= LOGIT_ATOL
    for i in range(6):
        tok = int(np.argmax(want))
        got, want = ex.decode(tok), dec.decode(tok)
        assert np.abs(got - want).max() <= LOGIT_ATOL, f"step {i}"
    eng.close()


@pytest.mark.gpu
def test_config2_full_workload_matches_oracle(gpu, orc):
    """Config 2 at its own workload: mla36m (Model::create seed 0, fp16 weights), one
    session, a 1024-id prompt from Rng(0).bounded(16384) prefilled as ONE 1024-row chunk,
    then 64 greedy decode calls, against the oracle's CpuDecoder on the same fp16 weights
    with an fp16-rounded cache (tests/test_mps.cpp:126-166 runs the same prefill / decode
    comparison at 0.015; LOGIT_ATOL here).  The decode tokens follow the oracle's greedy
    choice; the GPU's greedy token must equal it wherever the oracle's top-2 margin
    exceeds 2 * LOGIT_ATOL."""
    cfg, params, p16 = _models(MLA36M)
    prompt = _prompt(1024, MLA36M["vocab_size"], seed=0)
    eng = _engine(gpu, MLA36M, params, max_sessions=2, max_rows=1024, num_pages=20)
    ex = eng.session()
    dec = orc.Decoder(cfg, p16, round_cache=True)
    got, want = ex.prefill(prompt), dec.prefill(prompt)
    err = np.abs(got - want).max()
    _say(f"config2 prefill (1024 rows, one chunk) max |err| {err:.3e}")
    assert err <= LOGIT_ATOL
    worst, checked = err, 0
    for i in range(64):
        tok = int(np.argmax(want))
        if _margin_ok(want):
            assert int(np.argmax(got)) == tok, f"greedy token at step {i}"
            checked += 1
        got, want = ex.decode(tok), dec.decode(tok)
        err = np.abs(got - want).max()
        worst = max(worst, err)
        assert err <= LOGIT_ATOL, f"decode step {i}: {err}"
    assert ex.position == 1088
    _say(f"config2 64 decodes: max |err| {worst:.3e}, greedy tokens checked {checked}/64")
    eng.close()


@pytest.mark.gpu
def test_shorter_reprefill_after_decoding(gpu, orc):
    """tests/test_mps.cpp:158-165: an execution that has prefilled and decoded takes a new,
    shorter prompt; prefill restarts at position 0 and returns that prompt's logits."""
    cfg, params, p16 = _models(MLA36M, seed=9)
    eng = _engine(gpu, MLA36M, params, max_sessions=2, max_rows=64, num_pages=8)
    ex = eng.session()
    dec = orc.Decoder(cfg, p16, round_cache=True)
    tokens = [1, 5, 8]
    np.testing.assert_allclose(ex.prefill(tokens), dec.prefill(tokens), rtol=0, atol=LOGIT_ATOL)
    for i in range(14):
        t = (i * 3 + 2) % 32
        np.testing.assert_allclose(ex.decode(t), dec.decode(t), rtol=0, atol=LOGIT_ATOL)
    assert ex.position == 17
    free_before = eng.info()["free_pages"]
    got = ex.prefill([2, 3])
    assert ex.position == 2 and eng.info()["free_pages"] == free_before
    want = orc.forward(cfg, p16, [2, 3])[-1]
    np.testing.assert_allclose(got, want, rtol=0, atol=LOGIT_ATOL)
    np.testing.assert_allclose(ex.decode(4), orc.forward(cfg, p16, [2, 3, 4])[-1], rtol=0,
                               atol=LOGIT_ATOL)
    eng.close()


@pytest.mark.gpu
def test_weight_changes_invalidate_decode_cache(gpu, orc):
    """tests/test_training.cpp:111-122 on the engine: after the weights change, a session
    prefilled with the old ones cannot decode (invalid_argument, CpuDecoder's message,
    inference.cpp:71-75), nor can its fork; after a new prefill it decodes with the new
    weights, equal to the oracle on them."""
    import cpp_inference_train_engine_amd as mla
    cfg, params, _ = _models(TINY, seed=9)
    eng = _engine(gpu, TINY, params, max_sessions=4, max_rows=64, num_pages=16, page_size=16)
    a, empty = eng.session(), eng.session()
    a.prefill([1, 2, 3])
    a.decode(4)
    fork = a.fork_prefix()
    new = params.copy()
    new[0] += 0.01  # token_embedding[0, 0], as the reference test changes it
    new[1000:2000] *= 1.5
    eng.update_weights(new)
    assert eng.stats()["revision"] == 1
    for s in (a, fork):
        with pytest.raises(mla.MlaError) as e:
            s.decode(4)
        assert e.value.code == "invalid_argument"
        assert "current-weight prefill" in str(e.value)
        with pytest.raises(mla.MlaError):
            eng.step([s], [[4]])
    p16 = orc.bits_to_f32(orc.round_f16(new))
    dec = orc.Decoder(cfg, p16, round_cache=True)
    np.testing.assert_allclose(a.prefill([1, 2, 3]), dec.prefill([1, 2, 3]), rtol=0,
                               atol=LOGIT_ATOL)
    np.testing.assert_allclose(a.decode(4), dec.decode(4), rtol=0, atol=LOGIT_ATOL)
    # a session that held nothing when the weights changed starts on the new ones
    np.testing.assert_allclose(empty.prefill([1, 2, 3]), orc.Decoder(
        cfg, p16, round_cache=True).prefill([1, 2, 3]), rtol=0, atol=LOGIT_ATOL)
    eng.close()


@pytest.mark.gpu
def test_forward_returns_every_position(gpu, orc):
    """Execution::forward(ids, batch, sequence) (execution.hpp:38-39): the logits of every
    position of each sequence equal Model::forward's (the oracle's) rows; chunking by
    max_rows changes nothing; and decode after prefill equals forward's last row, the check
    the reference's decode bench records (apps/bench_main.cpp:378-396)."""
    cfg, params, p16 = _models(MLA36M, seed=6)
    rng = np.random.default_rng(6)
    ids = rng.integers(0, MLA36M["vocab_size"], (3, 70)).astype(np.uint16)
    eng = _engine(gpu, MLA36M, params, max_sessions=4, max_rows=256, num_pages=16)
    got = eng.forward(ids, 3, 70)
    assert got.shape == (210, MLA36M["vocab_size"])
    for b in range(3):
        want = orc.forward(cfg, p16, ids[b])
        err = np.abs(got[b * 70:(b + 1) * 70] - want).max()
        _say(f"forward sequence {b}: max |err| {err:.3e}")
        assert err <= LOGIT_ATOL
    assert eng.info()["active_sessions"] == 0 and eng.info()["free_pages"] == 16
    ex = eng.session()
    ex.prefill(ids[0, :69])
    np.testing.assert_allclose(ex.decode(int(ids[0, 69])), got[69], rtol=0, atol=LOGIT_ATOL)
    eng.close()
    small = _engine(gpu, MLA36M, params, max_sessions=4, max_rows=50, num_pages=16)
    np.testing.assert_allclose(small.forward(ids, 3, 70), got, rtol=0, atol=1e-5)
    small.close()


@pytest.mark.gpu
def test_stats_count_submissions_waits_and_kernels(gpu):
    """Execution::stats (execution.hpp:25-27, reported per update by bench_main.cpp:
    358-368): one decode call is one forward submission and one host wait; its kernels are
    the metadata build, the embedding, per layer the projections, the attention (one
    launch over XCD-placed metadata, else the decode kernel and its split merge) and the
    three FFN kernels, then the logits and the greedy token."""
    _, params, _ = _models(MLA36M, seed=7)
    eng = _engine(gpu, MLA36M, params, max_sessions=2, max_rows=64, num_pages=8)
    ex = eng.session()
    ex.prefill(list(range(1, 41)))
    before = ex.stats()
    ex.decode(5)
    after = ex.stats()
    L = MLA36M["n_layers"]
    assert after["graph_submissions"] - before["graph_submissions"] == 1
    assert after["host_waits"] - before["host_waits"] == 1
    per_layer = 5 if gpu.xcd_count() > 0 else 6
    assert after["kernel_submissions"] - before["kernel_submissions"] == 1 + 1 + per_layer * L + 2
    eng.close()


@pytest.mark.gpu
def test_decode_equals_full_recomputation_on_gpu(gpu):
    """tests/test_training.cpp:52-76 on the engine: after prefill(prompt) and k decodes,
    the logits equal those of prefill(prompt + the k tokens) (one chunk and 3 chunks)."""
    _, params, _ = _models(MLA36M, seed=2)
    prompt = _prompt(130, MLA36M["vocab_size"], seed=2)
    for max_rows in (256, 50):
        eng = _engine(gpu, MLA36M, params, max_sessions=2, max_rows=max_rows, num_pages=16)
        a, b = eng.session(), eng.session()
        logits = a.prefill(prompt)
        seq = list(prompt)
        for k in range(5):
            tok = int(np.argmax(logits))
            seq.append(tok)
            logits = a.decode(tok)
            full = b.prefill(seq)
            err = np.abs(logits - full).max()
            assert err <= LOGIT_ATOL, f"max_rows={max_rows} step {k}: {err}"
        eng.close()


@pytest.mark.gpu
def test_batched_step_equals_single_sessions(gpu):
    """One step mixing chunked prefills and decodes gives each session the logits it gets
    when stepped alone (rows are independent; the split of each session's pages is fixed)."""
    _, params, _ = _models(MLA36M, seed=3)
    eng = _engine(gpu, MLA36M, params, max_sessions=12, max_rows=512, num_pages=64)
    rng = np.random.default_rng(3)
    prompts = [rng.integers(0, 16384, int(n)).astype(np.uint16) for n in (70, 1, 130, 64, 5, 200)]
    solo, batch = [eng.session() for _ in prompts], [eng.session() for _ in prompts]
    solo_logits = [s.prefill(p) for s, p in zip(solo, prompts)]
    # the batch: sessions 0-2 prefilled alone first, then everything in one step
    for s, p in list(zip(batch, prompts))[:3]:
        s.prefill(p)
    nxt = [int(t) for t in rng.integers(0, 16384, 3)]
    chunks = [[nxt[0]], [nxt[1]], [nxt[2]]] + [list(p) for p in prompts[3:]]
    logits, greedy = eng.step(batch, chunks)
    for i, (s, ch) in enumerate(zip(solo, chunks)):
        want = s.decode(ch[0]) if i < 3 else solo_logits[i]
        np.testing.assert_allclose(logits[i], want, rtol=0, atol=1e-5, err_msg=f"session {i}")
        assert greedy[i] == int(np.argmax(want))
    eng.close()


@pytest.mark.gpu
def test_failed_fused_check_reruns_the_step_unplaced(gpu):
    """A placed step whose decode status comes back nonzero (forced from the host with
    mla_testing_fail_decode_status: the state a broken XCD placement leaves) is rerun by the
    engine through the two-launch decode: the same logits as an engine whose checks passed,
    one rerun counted, and placement off for the engine's later steps."""
    _, params, _ = _models(MLA36M, seed=5)
    prompts = [_prompt(n, 16384, seed=n) for n in (700, 1300, 90, 2000)]
    engines = [_engine(gpu, MLA36M, params, max_sessions=4, max_rows=4096, num_pages=120)
               for _ in range(2)]
    sess = [[e.session() for _ in prompts] for e in engines]
    for e, ss in zip(engines, sess):
        e.step(ss, [list(p) for p in prompts])
    nxt = [[11], [12], [13], [14]]
    want, _ = engines[0].step(sess[0], nxt)
    assert engines[0].stats()["fused_reruns"] == 0
    gpu.check(gpu.lib().mla_testing_fail_decode_status(1))
    try:
        _say("engine step with a failed fused check")
        got, _ = engines[1].step(sess[1], nxt)
    finally:
        gpu.check(gpu.lib().mla_testing_fail_decode_status(0))
    assert engines[1].stats()["fused_reruns"] == 1
    # The two-launch merge sums the partials in another order, and the step's fp16
    # activations carry that last-bit difference to the logits: the engines' parity bound.
    np.testing.assert_allclose(got, want, rtol=0, atol=LOGIT_ATOL)
    assert (np.argmax(got, 1) == np.argmax(want, 1)).all()
    want2, _ = engines[0].step(sess[0], [[21], [22], [23], [24]])
    got2, _ = engines[1].step(sess[1], [[21], [22], [23], [24]])
    assert engines[0].stats()["fused_reruns"] == 0 and engines[1].stats()["fused_reruns"] == 1
    np.testing.assert_allclose(got2, want2, rtol=0, atol=LOGIT_ATOL)
    for e in engines:
        e.close()


@pytest.mark.gpu
def test_fork_shares_pages_and_copies_on_write(gpu):
    """A forked session shares its source's pages; the first append into the shared
    partial page copies it, so both sessions continue as if prefilled separately."""
    _, params, _ = _models(MLA36M, seed=4)
    eng = _engine(gpu, MLA36M, params, max_sessions=6, max_rows=256, num_pages=32)
    prompt = _prompt(100, MLA36M["vocab_size"], seed=4)  # one full page + a partial one
    a = eng.session()
    a.prefill(prompt)
    free0 = eng.info()["free_pages"]
    b = a.fork_prefix()
    assert eng.info()["free_pages"] == free0 and b.position == 100
    la, lb = a.decode(7), b.decode(9)
    assert eng.info()["free_pages"] == free0 - 1  # b's copy of the shared partial page
    ra, rb = eng.session(), eng.session()
    np.testing.assert_allclose(la, ra.prefill(list(prompt) + [7]), rtol=0, atol=LOGIT_ATOL)
    np.testing.assert_allclose(lb, rb.prefill(list(prompt) + [9]), rtol=0, atol=LOGIT_ATOL)
    for s in (a, b, ra, rb):
        s.release()
    assert eng.info()["free_pages"] == 32
    eng.close()


@pytest.mark.gpu
def test_engine_errors_match_the_reference(gpu):
    import cpp_inference_train_engine_amd as mla
    _, params, _ = _models(TINY)
    eng = _engine(gpu, TINY, params, max_sessions=2, max_rows=16, num_pages=4, page_size=16)
    s = eng.session()
    with pytest.raises(mla.MlaError) as e:
        s.decode(1)  # no prefill yet (inference.cpp:71-75)
    assert e.value.code == "invalid_argument"
    with pytest.raises(mla.MlaError) as e:
        s.prefill([])
    assert e.value.code == "invalid_argument" and "Prompt exceeds context" in str(e.value)
    with pytest.raises(mla.MlaError):
        s.prefill(list(range(65)))  # > max_sequence_length 64
    s.prefill([1, 2, 3])
    with pytest.raises(mla.MlaError):
        s.decode(264)  # token >= vocab
    with pytest.raises(mla.MlaError) as e:  # one page left after the other session's 3
        t = eng.session()
        t.prefill(list(range(60)))
    assert e.value.code == "out_of_memory"
    assert t.position == 0 and eng.info()["free_pages"] == 3
    assert s.position == 3
    s.decode(5)
    assert s.position == 4
    with pytest.raises(mla.MlaError):
        eng.step([s, s], [[1], [2]])  # a session listed twice
    assert s.position == 4
    eng.close()


@pytest.mark.gpu
def test_sessions_on_threads_equal_serial_runs(gpu):
    """Three sessions decoded concurrently from threads, three repeats
    (tests/inference_sessions.hpp:191-217): each equals the serial run."""
    _, params, _ = _models(TINY, seed=5)
    eng = _engine(gpu, TINY, params, max_sessions=8, max_rows=64, num_pages=32, page_size=16)
    prompts = [_prompt(n, 264, seed=n) for n in (5, 9, 17)]

    def run(p, out, idx):
        ex = eng.session()
        logits = ex.prefill(p)
        seq = []
        for _ in range(12):
            t = int(np.argmax(logits))
            seq.append(t)
            logits = ex.decode(t)
        out[idx] = (seq, logits)
        ex.release()

    serial = [None] * 3
    for i, p in enumerate(prompts):
        run(p, serial, i)
    for _ in range(3):
        par = [None] * 3
        th = [threading.Thread(target=run, args=(p, par, i)) for i, p in enumerate(prompts)]
        for t in th:
            t.start()
        for t in th:
            t.join()
        for i in range(3):
            assert par[i][0] == serial[i][0]
            np.testing.assert_array_equal(par[i][1], serial[i][1])
    eng.close()
