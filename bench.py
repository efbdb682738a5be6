"""Benchmark of the MLA ragged decode hot path on one MI355X.

Workload ("config 3"): the mla36m model (10 blocks,
d=512, 8 MLA heads, q-rank 192, KV rank 128, tied 16384 vocab; random-init
weights with Model::create's scales, fp16 on the device), 64 sessions with
context lengths uniform in [128, 4096], one decode token each, fp16 paged latent
cache (64-token pages at a random page permutation), N(0,1) cache contents.

A timed step = one full batched decode step: the GPU metadata build, then
mla_model_step (token embedding; per layer RMSNorm, the q / kv projections with
the paged append, the W_uk absorption, the paged decode attention with its split
merge, the combined W_uv.W_o output projection, the SwiGLU FFN; final RMSNorm,
tied logits and the greedy token).  Each step feeds its greedy tokens back as the
next step's tokens; the positions stay those of config 3 (each replay rewrites the
same cache slots).  The step is captured once in a HIP graph and replayed; K
replays are timed between two synchronisations.  Inputs are resident in HBM.

The roofline block reports the dominant kernel of the path, decode_page_kernel
(one mla_decode_partials call per layer), launched back-to-back over the 10
layer pools in a graph and timed with HIP events on the stream the graph
replays on; `attention_call` reports the whole mla_decode_attention call
(+ merge_kernel) the same way.  `traffic` comes from the FETCH_SIZE /
WRITE_SIZE passes recorded under profiles/ (scaled by the same counters over a
plain copy of known size, run by --copy-probe-mib).

Prints ONE JSON line (driver contract).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
N_LAYERS = 10
TRAFFIC_FILE = os.path.join(REPO, "profiles", "pmc_decode_page_kernel_config3.txt")
TRAFFIC_FILE_FUSED = os.path.join(REPO, "profiles", "pmc_decode_page_kernel_fused_config3.txt")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--sessions", type=int, default=64)
    ap.add_argument("--target-blocks", type=int, default=1024)
    ap.add_argument("--split-pages", type=int, default=4)
    ap.add_argument("--kernel-reps", type=int, default=50,
                    help="graph replays of 20 back-to-back attention calls")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead")
    ap.add_argument("--no-placement", action="store_true",
                    help="work items in session order and a separate merge launch per layer")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the config-2, config-4 and config-5 legs")
    ap.add_argument("--cpu-seconds", type=float, default=5.0,
                    help="seconds of CPU timing per baseline leg (all cores, 1 thread; half "
                         "of it for the non-absorbed fallback)")
    ap.add_argument("--flags", type=int, default=0)
    ap.add_argument("--only", choices=["config2", "config4", "config5", "serve"], default=None,
                    help="run only this secondary leg and print its JSON (for profiling)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first run a plain device copy of this many MiB (counter calibration)")
    return ap.parse_args()


def traffic_from_profile(fused: bool = False):
    """HBM bytes per decode_page_kernel launch, as recorded by the counter passes (of the
    fused-merge instantiation when ``fused``)."""
    path = TRAFFIC_FILE_FUSED if fused else TRAFFIC_FILE
    try:
        with open(path) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", f.read(), re.M)
        return int(m.group(1)) if m else None
    except OSError:
        return None


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_it(warmup: int, reps: int, prepare, operation):
    """The reference's timing (apps/bench_main.cpp:12-30): `warmup` untimed runs, then
    `reps` timed ones, prepare() outside the clock; returns the sorted samples in ms."""
    samples = []
    for i in range(-warmup, reps):
        prepare()
        t0 = time.perf_counter()
        operation()
        dt = (time.perf_counter() - t0) * 1e3
        if i >= 0:
            samples.append(dt)
    return sorted(samples)


def median_p95(samples):
    """Median and p95 of sorted samples as bench_main.cpp:26-29 takes them (the element
    at n / 2, and at ceil(0.95 n) - 1)."""
    n = len(samples)
    return samples[n // 2], samples[min(n - 1, int(np.ceil(n * 0.95)) - 1)]


def cpu_baseline(batch, params, seconds: float, traces=None):
    """The reference CPU path for the same step: the oracle's fp32 restatement of
    CpuDecoder::decode (inference.cpp:69-174: projections, absorbed attention over the
    session's contiguous cache, FFN, tied logits), timed like apps/bench_main.cpp:12-30
    and 395-408: per decode call, with warmup, median and p95; `prepare` rewinds the
    session to its config-3 length.  A bounded sample of the batch's sessions (spread over
    its lengths) decodes one session per thread on every visible core (forks decode
    concurrently, inference.cpp:238), then the same sessions one after another on 1 thread,
    then with the non-absorbed K/V reconstruction (CpuDecoder::set_absorbed(false),
    bench_main.cpp:400-408: baseline_median_ms and speedup).  The products run on the CBLAS
    numpy ships (OpenBLAS, one thread per call) in place of the reference's Accelerate.

    `traces` (the GPU legs' inputs and outputs) are checked here, with the oracle as the
    checker, as the reference's benches record a correctness error next to each timing
    (bench_main.cpp:378-396)."""
    import threading
    import oracle
    from cpp_inference_train_engine_amd.workloads import MLA36M
    blas = oracle.use_blas(True)
    cfg = oracle.Config.from_dict(MLA36M)
    visible = len(os.sched_getaffinity(0))
    n_sess = max(1, min(visible, len(batch.k_len)))
    pick = np.argsort(batch.k_len)[np.linspace(0, len(batch.k_len) - 1, n_sess).astype(int)]
    proj = oracle.output_projection(cfg, params)  # prepare_projections, once per model

    def decoders(absorbed):
        out = []
        for b in pick:  # each sampled session at its config-3 length (cache contents N(0,1))
            d = oracle.Decoder(cfg, params, absorbed=absorbed, proj=proj)
            n = int(batch.ctx_len[b])
            gen = np.random.default_rng(int(b))
            d.latent[:, :n] = gen.standard_normal((cfg.n_layers, n, cfg.kv_lora_rank),
                                                  np.float32)
            d.rope[:, :n] = gen.standard_normal((cfg.n_layers, n, cfg.head_dim_rope),
                                                np.float32)
            out.append((d, n))
        return out

    def rewind(dn):
        dn[0].position = dn[1]

    decs = decoders(True)
    # Per-call cost estimate from one untimed call per session (sizes the repetitions).
    est = []
    for dn in decs:
        est.append(time_it(0, 1, lambda: rewind(dn), lambda: dn[0].decode(1))[0])
    longest = max(est) * 1e-3
    # all cores: one session per thread, `reps` timed calls each after 2 warmup calls
    reps = int(np.clip(seconds / longest, 5, 5000))
    samples, lock = [], threading.Lock()
    ready = threading.Barrier(len(decs) + 1)

    def worker(dn):
        time_it(2, 0, lambda: rewind(dn), lambda: dn[0].decode(1))
        ready.wait()
        got = time_it(0, reps, lambda: rewind(dn), lambda: dn[0].decode(1))
        with lock:
            samples.extend(got)

    threads = [threading.Thread(target=worker, args=(dn,)) for dn in decs]
    for t in threads:
        t.start()
    ready.wait()
    t0 = time.perf_counter()
    for t in threads:
        t.join()
    wall = time.perf_counter() - t0
    samples.sort()
    many_med, many_p95 = median_p95(samples)
    many = len(samples) / wall
    # 1 thread: the same sessions in turn
    per = max(2, int(seconds / (sum(est) * 1e-3)))
    one = []
    t0 = time.perf_counter()
    for dn in decs:
        one += time_it(1, per, lambda: rewind(dn), lambda: dn[0].decode(1))
    one.sort()
    one_med, one_p95 = median_p95(one)
    single = len(one) / sum(one) * 1e3
    # 1 thread, non-absorbed (the reference's fallback baseline)
    del decs
    base = []
    per_b = max(2, int(0.5 * seconds / (sum(est) * 1e-3)))
    for dn in decoders(False):
        base += time_it(1, per_b, lambda: rewind(dn), lambda: dn[0].decode(1))
    base.sort()
    base_med, base_p95 = median_p95(base)
    mean_ctx = float(np.mean(batch.ctx_len[pick]))
    out = {"value": round(many, 2), "unit": "tok/s", "cores": len(pick), "kind": "port",
           "timing": "time_it (apps/bench_main.cpp:12-30): per decode call, warmup untimed, "
                     "median and p95; value = timed calls / wall clock of the timed phase",
           "median_ms": round(many_med, 3), "p95_ms": round(many_p95, 3),
           "one_core": {"value": round(single, 2), "median_ms": round(one_med, 3),
                        "p95_ms": round(one_p95, 3), "calls": len(one)},
           "non_absorbed_one_core": {"baseline_median_ms": round(base_med, 3),
                                     "p95_ms": round(base_p95, 3), "calls": len(base),
                                     "speedup": round(base_med / one_med, 3)},
           "cpu_model": cpu_model(), "host_cores_visible": visible,
           "blas": f"{blas} (numpy's scipy_openblas64, standing in for Accelerate)"
                   if blas else "none found: unblocked C loops",
           "sample": f"full decode step (oracle CpuDecoder restatement, fp32) of {len(pick)} "
                     f"sessions spread over the batch's lengths (mean context {mean_ctx:.0f}): "
                     f"{len(samples)} timed calls on {len(pick)} threads, one session per "
                     f"thread; {len(one)} on 1 thread; {len(base)} non-absorbed on 1 thread"}
    traces = traces or {}
    acc = {}
    if "config2" in traces:
        acc["config2"] = check_config2(oracle, cfg, params, traces["config2"])
    if "config3" in traces:
        acc["config3"] = check_config3(oracle, cfg, params, batch, traces["config3"])
    if "config4" in traces:
        acc["config4"] = check_attention(oracle, traces["config4"], visible)
    if "config5" in traces:
        acc["config5"] = check_attention(oracle, traces["config5"], visible)
    out["accuracy"] = acc
    oracle.use_blas(False)
    return out


def check_config2(oracle, cfg, params, trace):
    """Config 2 replayed on the CPU path (1 thread): the same prompt and the GPU run's
    decode tokens on fp16-rounded weights and cache; the GPU logits' max error."""
    p16 = oracle.bits_to_f32(oracle.round_f16(params))
    d = oracle.Decoder(cfg, p16, round_cache=True)
    t0 = time.perf_counter()
    want = d.prefill(trace["prompt"])
    prefill_s = time.perf_counter() - t0
    pre_err = float(np.abs(trace["prefill_logits"] - want).max())
    dec_err, times = 0.0, []
    for tok, got in zip(trace["tokens"], trace["decode_logits"]):
        t0 = time.perf_counter()
        want = d.decode(int(tok))
        times.append(time.perf_counter() - t0)
        dec_err = max(dec_err, float(np.abs(got - want).max()))
    return {"prefill_max_abs_err": round(pre_err, 6), "decode_max_abs_err": round(dec_err, 6),
            "cpu_prefill_ms": round(prefill_s * 1e3, 1),
            "cpu_decode_ms_median": round(float(np.median(times)) * 1e3, 3),
            "sample": "config 2 replayed on the CPU path (1 thread): the same 1024-token "
                      "prompt and the GPU run's 64 decode tokens, fp16-rounded weights and "
                      "cache"}


def check_config3(oracle, cfg, params, batch, trace):
    """The timed config-3 step's logits for a sample of sessions against the CPU path's
    decode of the same token over the same cache words and fp16-rounded weights."""
    from cpp_inference_train_engine_amd.ops import latent_word, rope_word
    p16 = oracle.bits_to_f32(oracle.round_f16(params))
    proj = oracle.output_projection(cfg, p16)
    ps, kv, rp = batch.page_size, batch.kv_rank, batch.rope_dim
    lw = latent_word(np.arange(ps)[:, None], np.arange(kv)[None, :], ps, kv, rp)
    rw = rope_word(np.arange(ps)[:, None], np.arange(rp)[None, :], ps, kv, rp)
    err, greedy_same = 0.0, 0
    for b, got in zip(trace["sessions"], trace["logits"]):
        ids = batch.page_ids[batch.cu_pages[b]:batch.cu_pages[b + 1]]
        n = int(batch.ctx_len[b])
        t = np.arange(n)
        d = oracle.Decoder(cfg, p16, absorbed=True, round_cache=True, proj=proj)
        d.latent[:, :n] = oracle.bits_to_f32(batch.pages[:, ids[t // ps][:, None], lw[t % ps]])
        d.rope[:, :n] = oracle.bits_to_f32(batch.pages[:, ids[t // ps][:, None], rw[t % ps]])
        d.position = n
        want = d.decode(int(trace["tokens"][b]))
        err = max(err, float(np.abs(got - want).max()))
        greedy_same += int(np.argmax(got) == np.argmax(want))
    return {"logits_max_abs_err": round(err, 6), "sessions_checked": len(trace["sessions"]),
            "greedy_equal": greedy_same,
            "sample": "one more step of the benched graph's kernels after the timed loop; "
                      f"{len(trace['sessions'])} of the 64 sessions spread over the lengths, "
                      "each against the CPU path's decode (fp16 weights and cache words)"}


def check_attention(oracle, trace, threads):
    """Attention rows of a kernel leg against the oracle's paged attention over the same
    16-bit words: max |gpu - cpu| and the tolerance excess (north star: 2e-3 + 1e-3|x|)."""
    want = oracle.attention_paged(trace["H"], trace["kv"], trace["rope"], 64, trace["dtype"],
                                  trace["cu_q"], trace["k_len"], trace["table"], trace["pages"],
                                  oracle.bits_to_f32(trace["q_latent"], trace["dtype"]),
                                  oracle.bits_to_f32(trace["q_rope"], trace["dtype"]),
                                  trace["scale"], threads=threads)
    got = trace["out"]
    excess = float((np.abs(got - want) - (2e-3 + 1e-3 * np.abs(want))).max())
    return {"max_abs_err": round(float(np.abs(got - want).max()), 6),
            "max_tolerance_excess": round(excess, 6), "within_tolerance": excess <= 0,
            "rows_checked": int(got.shape[0]), "sample": trace["sample"]}


def config2_leg(mla, params, steps: int = 64, prompt_len: int = 1024):
    """Config 2: the mla36m model, one session, a 1024-token prompt (reference Rng seed 0,
    ids uniform in [0, vocab)), then 64 greedy decode steps through the session engine
    (mla_session_prefill / mla_session_decode: the reference's Execution::prefill and
    decode, logits returned to the host every step).  Times each decode call on the host
    clock like apps/bench_main.cpp:12-30 (median, p95).  Every decode's logits are then
    checked against the same backend's full forward of prompt + tokens (the reference's
    decode bench compares decode with Model::forward, bench_main.cpp:378-396).  Returns
    (record, trace): the trace (prompt, tokens, logits) lets the CPU-baseline leg measure
    the same logits against the CPU path."""
    from cpp_inference_train_engine_amd.workloads import MLA36M, SplitMix64
    cfg = mla.ModelConfig.from_dict(MLA36M)
    rng = SplitMix64(0)
    prompt = [rng.bounded(MLA36M["vocab_size"]) for _ in range(prompt_len)]
    eng = mla.HipEngine(cfg, params, max_sessions=2, max_rows=prompt_len, num_pages=48)
    ex = eng.session()
    ex.prefill(prompt)  # warm
    t0 = time.perf_counter()
    logits = ex.prefill(prompt)
    prefill_ms = (time.perf_counter() - t0) * 1e3
    trace = {"prompt": prompt, "prefill_logits": logits, "tokens": [], "decode_logits": []}
    times = []
    for _ in range(steps):
        tok = int(np.argmax(logits))
        t0 = time.perf_counter()
        logits = ex.decode(tok)
        times.append((time.perf_counter() - t0) * 1e3)
        trace["tokens"].append(tok)
        trace["decode_logits"].append(logits)
    st = ex.stats()
    full = eng.forward(prompt + trace["tokens"], 1, prompt_len + steps)
    fwd_err = float(np.abs(trace["prefill_logits"] - full[prompt_len - 1]).max())
    for i, got in enumerate(trace["decode_logits"]):
        fwd_err = max(fwd_err, float(np.abs(got - full[prompt_len + i]).max()))
    eng.close()
    med = float(np.median(times))
    rec = {"workload": "config 2: mla36m, one session, 1024-token prompt, 64 greedy decode "
                       "steps through the session engine (host-timed decode calls, logits "
                       "to host each step)",
           "prefill_ms": round(prefill_ms, 3), "decode_ms_median": round(med, 4),
           "decode_ms_p95": round(float(np.percentile(times, 95)), 4),
           "tok_per_s": round(1e3 / med, 1),
           "decode_vs_forward_max_abs_err": round(fwd_err, 6),
           "kernels_per_decode": round((st["kernel_submissions"]) / max(st["graph_submissions"], 1), 1),
           "reference_mps_fp16_ms": 3.583,
           "vs_reference_mps": round(3.583 / med, 2)}
    return rec, trace


def serve_leg(mla, params, temperature: float, requests: int = 64, new_tokens: int = 64):
    """Serving through the continuous-batching scheduler (mla_scheduler_*): the mla36m
    model, `requests` requests submitted at once, prompts of U[64, 512] ids (reference
    Rng seed 0, <|bos|> first), `new_tokens` tokens each (no stop), greedy (the device
    token) or sampled with the server's defaults (temperature 0.8, top_p 0.95, on the
    host from the step's logits).  Wall clock from the first submission to the last
    result; prompts are prefilled in chunks beside the running requests' decode rows."""
    from cpp_inference_train_engine_amd.workloads import MLA36M, SplitMix64
    cfg = mla.ModelConfig.from_dict(MLA36M)
    tok = mla.HipTokenizer(os.path.join(REPO, "tests", "golden", "tokenizer_pilot.json"))
    rng = SplitMix64(0)
    bos = tok.special("<|bos|>")
    prompts = [[bos] + [rng.bounded(256) for _ in range(64 + rng.bounded(449) - 1)]
               for _ in range(requests)]
    eng = mla.HipEngine(cfg, params, max_sessions=requests, max_rows=1024, num_pages=1024)
    gen = mla.GenerationConfig(max_new_tokens=new_tokens, temperature=temperature)
    out = {}
    with mla.Scheduler(eng, tok, max_context=2048, max_new_tokens=new_tokens,
                       max_queue=requests) as sch:
        sch.result(sch.submit(prompts[0][:8], gen))  # warm
        base = sch.metrics()
        t0 = time.perf_counter()
        ids = [sch.submit(p, gen) for p in prompts]
        res = [sch.result(i, timeout=300) for i in ids]
        wall = time.perf_counter() - t0
        m = sch.metrics()
    eng.close()
    done = sum(r["completion_tokens"] for r in res)
    out.update(workload=f"{requests} requests at once, prompts U[64,512] ids, {new_tokens} "
                        f"new tokens each, temperature {temperature}",
               wall_s=round(wall, 4), generated_tok_per_s=round(done / wall, 1),
               prompt_tokens=sum(len(p) for p in prompts), completion_tokens=done,
               steps=int(m["steps"] - base["steps"]),
               ms_per_step=round(wall * 1e3 / max(m["steps"] - base["steps"], 1), 4),
               mean_first_token_s=round(float(np.mean([r["first_token_seconds"] for r in res])), 4))
    return out


def config4_leg(mla, torch, reps: int = 20, n_pools: int = 4):
    """Config 4 (one layer, kernels only): 8 prefill chunks of 512 tokens on contexts
    U[0, 2048] + 120 decode sessions with log-normal lengths (median 2048, sigma 1, cap
    16384), half of the sessions aliasing a 256-token prefix.  Times the chunked-prefill
    kernel (MFMA-bound: flops = 544 per visible (query row, head, key)) and the decode
    attention call (HBM-bound: 288 B per cached token) with HIP events."""
    from cpp_inference_train_engine_amd.workloads import mixed_prefill_batch
    b = mixed_prefill_batch(seed=0)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    need = (b.k_len + 63) // 64
    mw = int(((need + 3) // 4).sum())
    rows = int(b.q_len.sum())
    # XCD-placed metadata (128 sessions): the decode call is one launch, merge included
    n_xcd = mla.xcd_count() if len(b.q_len) <= mla.PLACE_MAX_SESSIONS else 0
    if n_xcd:
        mw = mla.placed_work_slots(b.ctx_len, b.q_len, 64, 4, n_xcd)
    rb = mla.build_metadata(dev(b.ctx_len), dev(b.q_len), dev(b.cu_pages), dev(b.page_ids), 64,
                            b.max_pages, b.num_pages, split_pages=4, max_work=mw, max_rows=rows,
                            placement=n_xcd > 0)
    pages = dev(b.pages[0].view(np.int16)).view(torch.float16)
    # Copies of the layer's pool, visited in turn, so the working set (n_pools x ~120 MB)
    # exceeds the 256 MB Infinity Cache and every call reads HBM.
    pools = [pages] + [pages.clone() for _ in range(n_pools - 1)]
    ql = dev(b.q_latent.view(np.int16)).view(torch.float16)
    qr = dev(b.q_rope.view(np.int16)).view(torch.float16)
    out = torch.empty((rows, 8, 128), dtype=torch.float32, device="cuda")
    ws = mla.decode_workspace(mw, len(b.q_len), 8, 128)
    flops = sum(8 * 544 * (int(c) + i + 1) for c, q in zip(b.ctx_len, b.q_len) if q > 1
                for i in range(int(q)))
    dec_tokens = int(b.k_len[b.q_len == 1].sum())
    res = {}
    for kind in ("prefill", "decode"):
        def run(n):
            for i in range(n):
                pool = pools[i % n_pools]
                if kind == "prefill":
                    mla.prefill_attention(rb, pool, ql, qr, 0.125, kv_rank=128, rope_dim=16,
                                          max_q_len=512, out=out)
                else:
                    mla.decode_attention(rb, pool, ql, qr, 0.125, kv_rank=128, rope_dim=16,
                                         out=out, workspace=ws)
        run(3)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        run(reps)
        e1.record()
        torch.cuda.synchronize()
        res[kind] = e0.elapsed_time(e1) * 1e3 / reps
    rb.read_info()
    status = mla.decode_status(ws)
    tf = flops / res["prefill"] / 1e6
    gbs = dec_tokens * 288 / res["decode"] / 1e3
    pool_mb = pages.numel() * 2 / 1e6
    del pools
    # The last calls' rows (decode rows from the one-launch decode, prefill rows from the
    # chunked-prefill kernel) for the CPU leg's check, with the words they read.
    table = np.full((len(b.q_len), b.max_pages), -1, np.int32)
    for i in range(len(b.q_len)):
        lst = b.page_ids[b.cu_pages[i]:b.cu_pages[i + 1]]
        table[i, :len(lst)] = lst
    trace = {"H": 8, "kv": 128, "rope": 16, "dtype": 0, "scale": 0.125,
             "cu_q": np.concatenate([[0], np.cumsum(b.q_len)]).astype(np.int32),
             "k_len": b.k_len.astype(np.int32), "table": table, "pages": b.pages[0],
             "q_latent": b.q_latent, "q_rope": b.q_rope, "out": out.cpu().numpy(),
             "sample": "every row of the last timed calls (4,096 prefill rows, 120 decode "
                       "rows) against the oracle's paged attention"}
    return {"workload": "config 4 (one layer): 8 x 512-token chunks on contexts U[0,2048] + "
                        "120 log-normal decode sessions (median 2048, sigma 1, cap 16384), "
                        "4-page prefix shared by 64 sessions, fp16",
            "pools": f"{n_pools} copies of the layer's {pool_mb:.0f} MB pool visited in turn "
                     f"({n_pools * pool_mb:.0f} MB > the 256 MB Infinity Cache)",
            "prefill_kernel": {"us": round(res["prefill"], 2), "gflop": round(flops / 1e9, 3),
                               "tflops": round(tf, 1), "mfma_peak_tflops": 2500.0,
                               "frac": round(tf / 2500.0, 4)},
            "decode_call": {"us": round(res["decode"], 2), "cached_tokens": dec_tokens,
                            "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                            "one_launch": rb.placed, "fused_merge_status": status}}, trace


def config5_leg(mla, torch, reps: int = 5, split: int = 128):
    """Config 5 (kernel only): decode attention at the DeepSeek-like latent shape (128
    heads, kv_rank 512, rope 64, nope 128: scale 1/sqrt(192)), bf16 64-token pages, 256
    sessions with lengths U[8192, 32768] and the page permutation from the reference Rng
    (seed 0); cache and queries N(0, 1) drawn on the device (torch generator, seed 0).
    HBM bytes = 1152 per cached token; flops = 128 x (576 + 512) x 2 per cached token."""
    from cpp_inference_train_engine_amd.workloads import deepseek_decode_shape
    shape = deepseek_decode_shape(seed=0)
    gen = torch.Generator(device="cuda").manual_seed(0)
    pages = torch.randn((shape.num_pages, 64 * 576), generator=gen, device="cuda").to(
        torch.bfloat16)
    B = len(shape.k_len)
    ql = torch.randn((B, 128, 512), generator=gen, device="cuda").to(torch.bfloat16)
    qr = torch.randn((B, 128, 64), generator=gen, device="cuda").to(torch.bfloat16)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    need = (shape.k_len + 63) // 64
    mw = int(((need + split - 1) // split).sum())
    rb = mla.build_metadata(dev(shape.ctx_len), dev(shape.q_len), dev(shape.cu_pages),
                            dev(shape.page_ids), 64, shape.max_pages, shape.num_pages,
                            split_pages=split, max_work=mw)
    ws = mla.decode_workspace(mw, B, 128, 512)
    out = torch.empty((B, 128, 512), dtype=torch.float32, device="cuda")
    scale = 1.0 / np.sqrt(192.0)
    call = lambda: mla.decode_attention(rb, pages, ql, qr, scale, kv_rank=512, rope_dim=64,
                                        dtype=mla.DTYPE_BF16, out=out, workspace=ws)
    call()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        call()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    rb.read_info()
    tokens = int(shape.k_len.sum())
    gbs = tokens * 1152 / us / 1e3
    tf = tokens * 128 * 1088 * 2 / us / 1e6
    # 8 sessions spread over the length range (the shortest and the longest included), read
    # back with the pages they attend to, for the CPU leg's check.
    order = np.argsort(shape.k_len)
    picks = sorted(set(int(order[i]) for i in np.linspace(0, B - 1, 8).astype(int)))
    lists = [shape.page_ids[shape.cu_pages[i]:shape.cu_pages[i + 1]] for i in picks]
    flat = torch.from_numpy(np.concatenate(lists).astype(np.int64)).cuda()
    table = np.full((len(picks), max(len(x) for x in lists)), -1, np.int32)
    off = 0
    for i, x in enumerate(lists):
        table[i, :len(x)] = np.arange(off, off + len(x), dtype=np.int32)
        off += len(x)
    sel = torch.tensor(picks, device="cuda")
    bits = lambda t: t[sel].view(torch.int16).cpu().numpy().view(np.uint16)
    trace = {"H": 128, "kv": 512, "rope": 64, "dtype": 1, "scale": scale,
             "cu_q": np.arange(len(picks) + 1, dtype=np.int32),
             "k_len": shape.k_len[picks].astype(np.int32), "table": table,
             "pages": pages[flat].view(torch.int16).cpu().numpy().view(np.uint16),
             "q_latent": bits(ql), "q_rope": bits(qr), "out": out[sel].cpu().numpy(),
             "sample": f"{len(picks)} of the 256 sessions spread over the lengths "
                       f"({int(shape.k_len[picks].min())}..{int(shape.k_len[picks].max())} "
                       "tokens) against the oracle's paged attention"}
    del pages, ws
    return {"workload": "config 5 (kernel only): H=128, kv_rank 512, rope 64, bf16 64-token "
                        "pages, 256 sessions, len U[8192,32768], N(0,1) contents",
            "kernels": "decode_wide_kernel + merge_kernel (mla_decode_attention)",
            "split_pages": split, "work_items": mw, "cached_tokens": tokens,
            "us": round(us, 1), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "tflops": round(tf, 1), "mfma_frac": round(tf / 2500.0, 4)}, trace


def copy_probe(torch, mib: int):
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / 5
    print(f"# copy probe: {mib} MiB read + {mib} MiB written per launch, {us:.1f} us, "
          f"{2 * n / us / 1e3:.0f} GB/s", file=sys.stderr, flush=True)
    del src, dst


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the decode path shards by "
                                   "session (no cross-GPU exchange); --gpus must be 1"}))
        sys.exit(2)
    import torch
    import cpp_inference_train_engine_amd as mla
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch

    if args.copy_probe_mib > 0:
        copy_probe(torch, args.copy_probe_mib)
    from cpp_inference_train_engine_amd.workloads import MLA36M, model_params
    if args.only:
        legs = {"config2": lambda: config2_leg(mla, model_params(MLA36M, seed=0))[0],
                "config4": lambda: config4_leg(mla, torch)[0],
                "config5": lambda: config5_leg(mla, torch)[0],
                "serve": lambda: {"greedy": serve_leg(mla, model_params(MLA36M, seed=0), 0.0),
                                  "sampled": serve_leg(mla, model_params(MLA36M, seed=0), 0.8)}}
        print(json.dumps({args.only: legs[args.only]()}), flush=True)
        return
    t_gen = time.perf_counter()
    batch = ragged_decode_batch(B=args.sessions, n_layers=N_LAYERS, seed=0)
    params = model_params(MLA36M, seed=0)
    model = mla.HipModel(mla.ModelConfig.from_dict(MLA36M), params, max_batch=args.sessions)
    print(f"# workload and model ready in {time.perf_counter() - t_gen:.1f}s: "
          f"{int(batch.k_len.sum())} tokens/layer, {batch.num_pages} pages/layer", file=sys.stderr,
          flush=True)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    B, H = batch.q_latent.shape[:2]
    ctx_len, q_len = dev(batch.ctx_len), dev(batch.q_len)
    cu_pages, page_ids = dev(batch.cu_pages), dev(batch.page_ids)
    cache = mla.PagedLatentCache(N_LAYERS, batch.num_pages, 64, 128, 16, mla.DTYPE_F16,
                                 storage=dev(batch.pages.view(np.int16)).view(torch.float16))
    pools = [cache.layer(l) for l in range(N_LAYERS)]
    ql = dev(batch.q_latent.view(np.int16)).view(torch.float16)
    qr = dev(batch.q_rope.view(np.int16)).view(torch.float16)
    tokens = dev(np.random.default_rng(1).integers(0, MLA36M["vocab_size"], B).astype(np.int32))
    logits = torch.empty((B, MLA36M["vocab_size"]), dtype=torch.float32, device="cuda")
    # The host knows every session's length, so the work-item count is exact.  With XCD
    # placement the work list has the slots of the placed layout (empty ones included).
    pages_per_session = (batch.k_len + 63) // 64
    max_work = int(((pages_per_session + args.split_pages - 1) // args.split_pages).sum())
    n_xcd = 0 if args.no_placement or B > mla.PLACE_MAX_SESSIONS else mla.xcd_count()
    placed = n_xcd > 0
    if placed:
        max_work = mla.placed_work_slots(batch.ctx_len, batch.q_len, 64, args.split_pages, n_xcd)
    out = torch.empty((B, H, 128), dtype=torch.float32, device="cuda")
    ws = mla.decode_workspace(max_work, B, H, 128)
    scale = 1.0 / 8.0

    def meta():
        return mla.build_metadata(ctx_len, q_len, cu_pages, page_ids, 64, batch.max_pages,
                                  batch.num_pages, split_pages=args.split_pages,
                                  target_blocks=args.target_blocks, max_work=max_work,
                                  max_rows=B, placement=placed)

    def step():
        rb = meta()
        model.step(rb, tokens, ctx_len, pools, ws, logits=logits, next_tokens=tokens)
        return rb

    rb = step()
    info = rb.read_info()  # raises on a metadata error
    torch.cuda.synchronize()

    def attn_calls(n, fn, fused):
        for i in range(n):
            fn(rb, cache.layer(i % N_LAYERS), ql, qr, scale, kv_rank=128, rope_dim=16, out=out,
               workspace=ws, flags=args.flags, fused=fused)

    calls_per_replay = 2 * N_LAYERS
    # partials: the decode kernel without the merge; attention: the call as the step makes
    # it (one launch over placed metadata); two_launch: decode kernel + merge_kernel
    kinds = {"partials": (mla.decode_partials, False), "attention": (mla.decode_attention, placed),
             "two_launch": (mla.decode_attention, False)}
    if args.no_graph:
        run_step = step
        runners = {k: (lambda f=f: attn_calls(calls_per_replay, *f)) for k, f in kinds.items()}
    else:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):  # warm the allocator outside capture
            step()
            attn_calls(1, mla.decode_attention, placed)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g_step = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_step):
            step()
        runners = {}
        for k, f in kinds.items():
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                attn_calls(calls_per_replay, *f)
            runners[k] = g
        run_step = g_step.replay
        runners = {k: g.replay for k, g in runners.items()}

    for _ in range(args.warmup):
        run_step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        run_step()
    t1.record()
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / args.steps

    # Per-launch time of the dominant kernel (decode_page_kernel, one mla_decode_partials
    # call) and of the whole attention call (+ merge_kernel), each from back-to-back calls
    # over the 10 layer pools (389 MB working set > the 256 MB Infinity Cache), timed with
    # HIP events on the stream the graphs replay on.
    us = {}
    for k, run in runners.items():
        run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.kernel_reps):
            run()
        e1.record()
        torch.cuda.synchronize()
        us[k] = e0.elapsed_time(e1) * 1e3 / (args.kernel_reps * calls_per_replay)
    rb.read_info()
    # One more step of the same kernels, eager, for the CPU leg's check of the logits.
    step_tokens = tokens.cpu().numpy().copy()
    rb = step()
    torch.cuda.synchronize()
    # Every fused merge of the timed steps, the attention replays and this step found its
    # premises (the workspace's status word is sticky until cleared), else no number here
    # is trusted.
    status = mla.decode_status(ws)
    if status:
        raise SystemExit(f"decode status {status}: a fused merge's check failed; rerun with "
                         "--no-placement")
    sample3 = np.argsort(batch.k_len)[np.linspace(0, B - 1, 16).astype(int)]
    trace3 = {"tokens": step_tokens, "sessions": [int(b) for b in sample3],
              "logits": logits[torch.from_numpy(sample3).cuda()].cpu().numpy()}
    bytes_layer = batch.cache_bytes_per_layer()
    gbs = {k: bytes_layer / (v * 1e-6) / 1e9 for k, v in us.items()}
    # The dominant kernel as the step runs it: with placement, decode_page_kernel with the
    # split merge inside (the whole attention of a layer in one launch).
    main_k = "attention" if placed else "partials"
    achieved = gbs[main_k]
    result = {
        "metric": "MLA decode tok/s + attn-kernel HBM GB/s (% of peak), 64 ragged sessions",
        "value": round(B / (ms_step * 1e-3), 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 weights/cache/MFMA operands, f32 accumulate",
        "data": "synthetic",
        "config": {"workload": "config 3: mla36m (10 layers, d=512, 8 MLA heads, q-rank 192, "
                               "KV rank 128, tied 16384 vocab), random-init fp16 weights, 64 "
                               "ragged sessions, len U[128,4096], fp16 64-token pages; step = "
                               "metadata + full decode step (projections, paged append, "
                               "attention, FFN, logits, greedy), one HIP graph",
                   "sessions": B, "cached_tokens_per_layer": int(batch.k_len.sum()),
                   "split_pages": info[1], "work_items": info[0],
                   "xcd_placement": placed, "work_slots": max_work,
                   "fused_merge_status": status,
                   "cache_bytes": int(cache.pages.numel()) * 2,
                   "cache_bytes_read_per_step": N_LAYERS * bytes_layer,
                   "cache_bytes_note": "cache_bytes: the 10 layer page pools (64-token fp16 "
                                       "pages); the reference's decode record gives "
                                       "n_layers x max_sequence_length x kv_width x 2 per "
                                       "session (bench_main.cpp:410-415), "
                                       f"{N_LAYERS * MLA36M['max_sequence_length'] * 144 * 2} "
                                       "B for this model",
                   "timing": "eager" if args.no_graph else "hip graph"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profile(placed),
                     "kernel": ("decode_page_kernel<..., fused merge> (mla_decode_attention over "
                                "XCD-placed metadata: a layer's whole attention, split merge "
                                "included, in one launch)" if placed else
                                "decode_page_kernel (mla_decode_partials, one layer)"),
                     "us_per_launch": round(us[main_k], 3), "bytes_per_launch": bytes_layer},
        "decode_kernel_without_merge": {
            "kernel": "decode_page_kernel (mla_decode_partials: split partials left for a merge)",
            "us": round(us["partials"], 3), "GB/s": round(gbs["partials"], 1),
            "frac": round(gbs["partials"] / HBM_PEAK_GBS, 4)},
        "attention_two_launches": {
            "kernels": "decode_page_kernel + merge_kernel (mla_decode_attention without the "
                       "fused merge)",
            "us": round(us["two_launch"], 3), "GB/s": round(gbs["two_launch"], 1),
            "frac": round(gbs["two_launch"] / HBM_PEAK_GBS, 4)},
    }
    model.close()
    traces = {"config3": trace3}
    if not args.no_secondary:
        result["config2"], traces["config2"] = config2_leg(mla, params)
        result["config4"], traces["config4"] = config4_leg(mla, torch)
        result["config5"], traces["config5"] = config5_leg(mla, torch)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(batch, params, args.cpu_seconds, traces)
        # The CPU path's verdict on each timed leg's outputs, beside its timing.
        acc = result["cpu_baseline"].pop("accuracy")
        result["accuracy"] = acc.pop("config3")
        if "config2" in acc:
            c2 = acc.pop("config2")
            result["config2"]["decode_max_abs_err"] = c2["decode_max_abs_err"]
            result["config2"]["prefill_max_abs_err"] = c2["prefill_max_abs_err"]
            result["config2"]["cpu_path"] = c2
        for k, v in acc.items():
            result[k]["accuracy"] = v
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
