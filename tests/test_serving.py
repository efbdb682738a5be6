"""Generation and serving on the GPU: the device greedy token with banned ids, the
generation loop over engine sessions, and the continuous-batching scheduler
(mla_scheduler_*), with the reference's tiny-test weights and tokenizer.

Checks: the device's greedy token equals sample_token's greedy rule (oracle) on the
same logits with the same banned ids; generation over a session equals the oracle's
generate_tokens replayed on the logits the session produced; every request served by
the scheduler's batched steps gets exactly the tokens, text and finish reason that the
same request gets alone on a private session (the reference server's per-worker
result); the server's limits, queue bound, deadline, cancellation and metrics.
"""
import os
import time

import numpy as np
import pytest

from conftest import GOLDEN, TINY
from oracle import generation as og

TOK_TINY = os.path.join(GOLDEN, "tokenizer_tiny.json")
pytestmark = pytest.mark.gpu


def _engine(gpu, tiny_fixture, sessions=8):
    return gpu.HipEngine(gpu.ModelConfig.from_dict(TINY), tiny_fixture["params"],
                         max_sessions=sessions, max_rows=64, num_pages=64, page_size=16)


def _cfg(c):
    return dict(max_new_tokens=c.max_new_tokens, top_k=c.top_k, temperature=c.temperature,
                top_p=c.top_p, repetition_penalty=c.repetition_penalty, seed=c.seed,
                stop=c.stop, stop_tokens=c.stop_tokens)


def test_device_greedy_skips_banned_ids(gpu, tiny_fixture):
    eng = _engine(gpu, tiny_fixture)
    t = gpu.HipTokenizer(TOK_TINY)
    prompt = [t.special("<|bos|>")] + list(b"Hello")
    a, b = eng.session(), eng.session()
    logits_a, next_a = eng.step([a], [prompt])
    assert next_a[0] == og.sample_token(logits_a[0], [], og_cfg(0.0), og.Rng(0))
    banned = gpu.banned_tokens(t) + [int(next_a[0])]
    eng.set_banned(banned)
    logits_b, next_b = eng.step([b], [prompt])
    assert np.array_equal(logits_a, logits_b)
    assert next_b[0] == og.sample_token(logits_b[0], [], og_cfg(0.0), og.Rng(0), banned)
    assert next_b[0] != next_a[0]
    c = eng.session()
    eng.set_banned(list(range(TINY["vocab_size"])))
    with pytest.raises(gpu.MlaError) as e:
        eng.step([c], [prompt])
    assert e.value.code == "invalid_argument" and "All tokens are banned" in str(e.value)
    eng.set_banned([])
    _, next_c = eng.step([c], [[65]])
    assert next_c[0] >= 0
    eng.close()


def og_cfg(temperature, **kw):
    d = dict(max_new_tokens=16, top_k=0, temperature=temperature, top_p=0.95,
             repetition_penalty=1.0, seed=42, stop=(), stop_tokens=())
    d.update(kw)
    return d


class _Recorder:
    """Wraps an execution and keeps every logits vector it returned."""

    def __init__(self, ex):
        self.ex, self.seen = ex, []
        self.max_sequence_length = ex.max_sequence_length

    def prefill(self, ids):
        self.seen.append(np.array(self.ex.prefill(ids)))
        return self.seen[-1]

    def decode(self, token):
        self.seen.append(np.array(self.ex.decode(token)))
        return self.seen[-1]


def test_generation_on_the_engine(gpu, tiny_fixture):
    """<|bos|> + encode(prompt) on an engine session, greedy and sampled: the oracle's
    generate_tokens replayed on the logits the session returned gives the same tokens,
    text and finish reason (and asks for the same decodes)."""
    eng = _engine(gpu, tiny_fixture)
    t = gpu.HipTokenizer(TOK_TINY)
    G = gpu.GenerationConfig
    tb = [t.decode([i]) for i in range(t.vocab_size)]
    for c in (G(max_new_tokens=12, temperature=0), G(max_new_tokens=20, seed=7),
              G(max_new_tokens=20, temperature=1.2, top_k=20, repetition_penalty=1.3, seed=3,
                stop=("e",))):
        rec = _Recorder(eng.session())
        out = gpu.generate(rec, t, "Say hi.", c)
        replay = list(rec.seen)
        calls = []

        def prefill(ids):
            calls.append(("prefill", ids))
            return replay.pop(0)

        def decode(tok):
            calls.append(("decode", tok))
            return replay.pop(0)

        ids = [t.special("<|bos|>")] + list(b"Say hi.")
        want = og.generate_tokens(prefill, decode, tb, t.special("<|eos|>"), ids, _cfg(c),
                                  TINY["max_sequence_length"])
        assert not replay
        assert (out["tokens"], out["text"], out["finish_reason"]) == \
            (want["tokens"], want["text"], want["finish_reason"])
        rec.ex.release()
    eng.close()


def _requests(gpu, t):
    G = gpu.GenerationConfig
    rng = np.random.default_rng(0)
    out = []
    for k in range(10):
        prompt = [t.special("<|bos|>")] + rng.integers(32, 127, int(rng.integers(1, 30))).tolist()
        c = G(max_new_tokens=int(rng.integers(1, 24)),
              temperature=[0.0, 0.8, 1.3][k % 3], top_k=[0, 0, 16][k % 3],
              repetition_penalty=[1.0, 1.0, 1.2, 1.0, 0.9][k % 5], seed=100 + k,
              stop=(("a",) if k % 4 == 1 else ()))
        out.append((prompt, c, k % 2 == 0))
    return out


def test_scheduler_matches_private_sessions(gpu, tiny_fixture):
    """Ten concurrent requests (greedy and sampled, streamed and not, prompts of 1 to 30
    tokens, max_rows 64 so prompts are chunked beside decode rows) through one
    scheduler: each result equals generate_ids of the same request on a private
    session."""
    eng = _engine(gpu, tiny_fixture, sessions=6)
    t = gpu.HipTokenizer(TOK_TINY)
    reqs = _requests(gpu, t)
    with gpu.Scheduler(eng, t, max_context=64, max_new_tokens=32, max_queue=16) as sch:
        ids = [sch.submit(p, c, stream=s) for p, c, s in reqs]
        got = [sch.result(i, timeout=60) for i in ids]
        m = sch.metrics()
        text = sch.metrics_text()
    assert m["completed"] == len(reqs) and m["requests"] == len(reqs)
    assert m["generated_tokens"] == sum(len(g["tokens"]) for g in got)
    assert m["steps"] < sum(len(g["tokens"]) for g in got)  # requests shared steps
    for line in ("mini_mla_requests_total 10\n", "mini_mla_completed_total 10\n",
                 "mini_mla_rejected_total 0\n", "mini_mla_first_token_seconds_sum ",
                 "mini_mla_queue_depth 0\n"):
        assert line in text
    for (p, c, stream), g in zip(reqs, got):
        private = eng.session()
        chunks = []
        alone = gpu.generate_ids(private, t, p, c, callback=lambda s: chunks.append(s) or True)
        private.release()
        # a streamed request's text is its chunks, each cleaned on its own
        want_text = "".join(chunks) if stream else alone["text"]
        assert (g["tokens"], g["text"], g["finish_reason"]) == \
            (alone["tokens"], want_text, alone["finish_reason"]), (p, c)
        assert g["prompt_tokens"] == len(p) and g["completion_tokens"] == len(g["tokens"])
    eng.close()


def test_scheduler_limits_queue_deadline_cancel(gpu, tiny_fixture):
    eng = _engine(gpu, tiny_fixture, sessions=2)
    t = gpu.HipTokenizer(TOK_TINY)
    G = gpu.GenerationConfig
    prompt = [t.special("<|bos|>")] + list(b"Hi")
    with pytest.raises(gpu.MlaError) as e:
        gpu.Scheduler(eng, t, max_context=65)  # beyond max_sequence_length
    assert "Invalid server limits" in str(e.value)
    with gpu.Scheduler(eng, t, max_context=64, max_new_tokens=16, max_queue=2,
                       request_timeout_seconds=1) as sch:
        for bad, msg in ((G(max_new_tokens=17), "Request exceeds context or token limit"),
                         (G(temperature=-1), "Invalid generation settings"),
                         (G(top_p=0), "Invalid generation settings")):
            with pytest.raises(gpu.MlaError) as e:
                sch.submit(prompt, bad)
            assert e.value.code == "invalid_argument" and msg in str(e.value)
        # The server's default budget: min(max_new_tokens, max_context - prompt).
        r = sch.result(sch.submit(prompt, G(temperature=0), max_tokens_given=False))
        assert r["finish_reason"] in ("length", "stop") and len(r["tokens"]) <= 16
        held = [eng.session(), eng.session()]  # every slot taken: nothing can start
        first = sch.submit(prompt, G(temperature=0, max_new_tokens=4))
        second = sch.submit(prompt, G(temperature=0, max_new_tokens=4))
        with pytest.raises(gpu.MlaError) as e:
            sch.submit(prompt, G(temperature=0, max_new_tokens=4))
        assert e.value.code == "unavailable" and "Request queue is full" in str(e.value)
        sch.cancel(second)
        time.sleep(1.3)  # past the deadline of both
        for h in held:
            h.release()
        _, st = sch.poll(first, 5.0)
        assert st["done"] and st["error"] == 7 and \
            "Request queue deadline exceeded" in st["error_message"]
        _, st = sch.poll(second, 5.0)
        assert st["done"] and st["error"] == 0 and st["finish_reason"] == "cancelled"
        r = sch.result(sch.submit(prompt, G(temperature=0, max_new_tokens=4)))
        assert r["completion_tokens"] >= 1
        m = sch.metrics()
        assert (m["rejected"], m["errors"], m["completed"]) == (1, 3, 2)
    eng.close()


def test_scheduler_from_many_threads(gpu, tiny_fixture):
    """Submitters and pollers on several host threads at once (the server's accept loop
    and its clients): every request's result equals the same request run alone."""
    import threading
    eng = _engine(gpu, tiny_fixture, sessions=4)
    t = gpu.HipTokenizer(TOK_TINY)
    reqs = _requests(gpu, t) * 2  # 20 requests, 4 sessions: most of them queue
    results = [None] * len(reqs)
    errors = []
    with gpu.Scheduler(eng, t, max_context=64, max_new_tokens=32, max_queue=32) as sch:
        def client(k0):
            try:
                for k in range(k0, len(reqs), 4):
                    p, c, stream = reqs[k]
                    results[k] = sch.result(sch.submit(p, c, stream=stream), timeout=60)
            except Exception as e:  # reported below, with the thread's request
                errors.append((k0, repr(e)))
        threads = [threading.Thread(target=client, args=(k0,)) for k0 in range(4)]
        for th in threads:
            th.start()
        for th in threads:
            th.join(120)
        assert not any(th.is_alive() for th in threads)
        m = sch.metrics()
    assert not errors, errors
    assert m["completed"] == len(reqs) and m["rejected"] == 0
    for (p, c, stream), g in zip(reqs, results):
        private = eng.session()
        chunks = []
        alone = gpu.generate_ids(private, t, p, c, callback=lambda s: chunks.append(s) or True)
        private.release()
        want_text = "".join(chunks) if stream else alone["text"]
        assert (g["tokens"], g["text"], g["finish_reason"]) == \
            (alone["tokens"], want_text, alone["finish_reason"]), (p, c)
    eng.close()


@pytest.mark.gpu
def test_close_while_other_threads_poll(gpu, tiny_fixture):
    """A server shutting down while its handler threads poll: close() stops the scheduler
    (queued requests never start, running ones end as cancelled), wakes the waiting polls
    and frees it only after every call in progress has returned.  Each poller ends with a
    finished status or the scheduler's "closed" error, never a crash or a hang."""
    import threading
    eng = _engine(gpu, tiny_fixture, sessions=2)
    t = gpu.HipTokenizer(TOK_TINY)
    sch = gpu.Scheduler(eng, t, max_context=64, max_new_tokens=40, max_queue=16)
    cfg = gpu.GenerationConfig(max_new_tokens=40, temperature=0.0)
    rids = [sch.submit([t.special("<|bos|>")] + [5 + k] * 8, cfg, stream=True)
            for k in range(6)]
    outcomes, started = {}, threading.Barrier(len(rids) + 1)

    def poller(rid):
        started.wait()
        try:
            while True:
                _, status = sch.poll(rid, 0.5)
                if status["done"]:
                    outcomes[rid] = ("done", status["finish_reason"])
                    return
        except gpu.MlaError as e:
            outcomes[rid] = ("error", e.code)

    threads = [threading.Thread(target=poller, args=(r,)) for r in rids]
    for th in threads:
        th.start()
    started.wait()
    sch.close()
    for th in threads:
        th.join(30)
    assert not any(th.is_alive() for th in threads)
    assert set(outcomes) == set(rids)
    for kind, what in outcomes.values():
        assert (kind == "done" and what in ("stop", "length", "cancelled")) or \
            (kind == "error" and what == "unavailable"), (kind, what)
    with pytest.raises(gpu.MlaError):
        sch.submit([1, 2, 3], cfg)
    sch.close()  # idempotent
    eng.close()
