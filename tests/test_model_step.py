"""The batched decode step (mla_model_*) against the oracle's CpuDecoder restatement.

CPU: ModelConfig validation and parameter counts (src/model/config.cpp:7-48,
tests/test_model.cpp:21-28 known answers).

GPU: one step for B sessions with random fp16 caches of different lengths, compared
with oracle.Decoder (absorbed, fp16-rounded cache, inference.cpp:69-174) run per
session on the same fp16-rounded weights and cache rows.  The GPU rounds the
activations feeding every projection to fp16 (as the reference's fp16 MPS path does)
and keeps q_latent in the cache dtype (mps_backend.mm:561), so logits agree to
LOGIT_ATOL; the reference records 3.5e-3 to 3.9e-3 max-abs logit error for its own
fp16 GPU decode against its CPU path (docs/benchmarks/throughput-followup/
inference.json).  Appended cache rows agree to CACHE_ATOL + CACHE_RTOL*|x|; greedy
tokens are equal wherever the oracle's top-2 margin exceeds twice LOGIT_ATOL.
"""
import sys

import numpy as np
import pytest

from conftest import MLA36M, TINY

LOGIT_ATOL = 5e-3
CACHE_ATOL, CACHE_RTOL = 2e-2, 1e-2


def _cfg(d, **over):
    import cpp_inference_train_engine_amd as mla
    d = dict(d, **over)
    return mla.ModelConfig.from_dict(d)


# ------------------------------------------------------------------ CPU ----
def test_parameter_counts_match_reference_known_answers():
    import cpp_inference_train_engine_amd as mla
    assert mla.config_parameter_count(_cfg(MLA36M)) == 35_763_840
    assert mla.config_parameter_count(_cfg(TINY)) == 26_704
    mla.config_validate(_cfg(MLA36M))
    mla.config_validate(_cfg(TINY))


@pytest.mark.parametrize("over, words", [
    (dict(head_dim_rope=3), "odd RoPE"),
    (dict(d_model=30), "divisibility"),
    (dict(n_heads=0), "n_heads must be in [1, 65535]"),
    (dict(vocab_size=70000), "vocab_size must be in [1, 65535]"),
    (dict(n_layers=129), "layer"),
    (dict(norm_epsilon=0.0), "epsilon"),
    (dict(rope_theta=1.0), "theta"),
    (dict(d_model=65535, n_heads=1, d_ff=65535, n_layers=100), "one billion"),
])
def test_invalid_configs_are_rejected_like_the_reference(over, words):
    import cpp_inference_train_engine_amd as mla
    with pytest.raises(mla.MlaError) as e:
        mla.config_validate(_cfg(MLA36M, **over))
    assert e.value.code == "invalid_argument" and words in str(e.value)


def test_config_from_reference_json_keys():
    import json
    import cpp_inference_train_engine_amd as mla
    d = dict(MLA36M, model_type="mla_dense_decoder", version=1, norm="rmsnorm")
    c = mla.ModelConfig.from_dict(json.loads(json.dumps(d)))
    assert c.to_dict()["kv_lora_rank"] == 128 and c.qk_dim == 64
    with pytest.raises(ValueError):
        mla.ModelConfig.from_dict({k: v for k, v in MLA36M.items() if k != "d_ff"})


# ------------------------------------------------------------------ GPU ----
def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _dev(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _step_case(cfgd, B, max_ctx, seed, page_size=64):
    """Random model (reference init, seed), B sessions with ctx lengths in [1, max_ctx] and
    N(0,1) fp16 caches; returns GPU and oracle results."""
    import torch
    import oracle
    import cpp_inference_train_engine_amd as mla
    from cpp_inference_train_engine_amd.ops import latent_word, rope_word
    ocfg = oracle.Config.from_dict(cfgd)
    params = oracle.bits_to_f32(oracle.round_f16(oracle.model_init(ocfg, seed)))
    L, kv, rp, V = ocfg.n_layers, ocfg.kv_lora_rank, ocfg.head_dim_rope, ocfg.vocab_size
    rng = np.random.default_rng(seed)
    ctx = rng.integers(1, max_ctx + 1, size=B).astype(np.int32)
    tokens = rng.integers(0, V, size=B).astype(np.int32)
    # page lists with room for the appended token, physical ids permuted
    need = (ctx + 1 + page_size - 1) // page_size
    P = int(need.sum())
    perm = rng.permutation(P).astype(np.int32)
    cu_pages = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    rec = page_size * (kv + rp)
    pages = np.zeros((L, P, rec), np.uint16)
    lat = [oracle.round_f16(rng.standard_normal((L, c, kv), dtype=np.float32)) for c in ctx]
    rop = [oracle.round_f16(rng.standard_normal((L, c, rp), dtype=np.float32)) for c in ctx]
    for b in range(B):
        t = np.arange(ctx[b])
        pg = perm[cu_pages[b] + t // page_size]
        slot = t % page_size
        r = np.arange(kv)
        c = np.arange(rp)
        lw = latent_word(slot[:, None], r[None, :], page_size, kv, rp)
        rw = rope_word(slot[:, None], c[None, :], page_size, kv, rp)
        for l in range(L):
            pages[l, pg[:, None], lw] = lat[b][l]
            pages[l, pg[:, None], rw] = rop[b][l]
    model = mla.HipModel(mla.ModelConfig.from_dict(cfgd), params, max_batch=B,
                         page_size=page_size)
    rb = mla.build_metadata(_dev(ctx), _dev(np.ones(B, np.int32)), _dev(cu_pages), _dev(perm),
                            page_size, int(need.max()), P, split_pages=4)
    gpu_pages = [_dev(pages[l].view(np.int16)).view(torch.float16) for l in range(L)]
    ws = mla.decode_workspace(rb.max_work, B, ocfg.n_heads, kv)
    logits, nxt = model.step(rb, _dev(tokens), _dev(ctx), gpu_pages, ws)
    torch.cuda.synchronize()
    rb.read_info()
    got_pages = np.stack([p.view(torch.int16).cpu().numpy().view(np.uint16) for p in gpu_pages])
    model.close()
    want_logits, want_lat, want_rope, got_lat, got_rope = [], [], [], [], []
    for b in range(B):
        dec = oracle.Decoder(ocfg, params, absorbed=True, round_cache=True)
        dec.latent[:, :ctx[b]] = oracle.bits_to_f32(lat[b])
        dec.rope[:, :ctx[b]] = oracle.bits_to_f32(rop[b])
        dec.position = int(ctx[b])
        want_logits.append(dec.decode(int(tokens[b])))
        want_lat.append(dec.latent[:, ctx[b]].copy())
        want_rope.append(dec.rope[:, ctx[b]].copy())
        pg = perm[cu_pages[b] + ctx[b] // page_size]
        slot = ctx[b] % page_size
        got_lat.append(oracle.bits_to_f32(
            got_pages[:, pg, latent_word(slot, np.arange(kv), page_size, kv, rp)]))
        got_rope.append(oracle.bits_to_f32(
            got_pages[:, pg, rope_word(slot, np.arange(rp), page_size, kv, rp)]))
    return dict(logits=logits.cpu().numpy(), next=nxt.cpu().numpy(),
                want_logits=np.stack(want_logits), lat=np.stack(got_lat),
                want_lat=np.stack(want_lat), rope=np.stack(got_rope),
                want_rope=np.stack(want_rope))


def _check_step(r, what):
    err = np.abs(r["logits"] - r["want_logits"]).max()
    lat_exc = (np.abs(r["lat"] - r["want_lat"]) - (CACHE_ATOL + CACHE_RTOL * np.abs(r["want_lat"]))).max()
    rope_exc = (np.abs(r["rope"] - r["want_rope"]) - (CACHE_ATOL + CACHE_RTOL * np.abs(r["want_rope"]))).max()
    _say(f"{what}: max |logit err| {err:.3e}, latent excess {lat_exc:.3e}, rope excess {rope_exc:.3e}")
    assert err <= LOGIT_ATOL, f"{what}: logits max abs error {err}"
    assert lat_exc <= 0 and rope_exc <= 0, f"{what}: appended cache rows"
    want = r["want_logits"]
    top2 = np.sort(want, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2 * LOGIT_ATOL
    ref_tok = np.argmax(want, axis=1)  # numpy argmax: lowest index among the maxima
    assert (r["next"][clear] == ref_tok[clear]).all(), f"{what}: greedy tokens"
    assert (r["next"] >= 0).all()


def _config3_case(seed=0, placement=False):
    """Config 3 exactly as bench.py times it: mla36m (max_sequence_length 4608) with
    Model::create-scaled weights from the oracle (seed 0, fp16), 64 sessions whose lengths
    after the append are U[128, 4096] (ragged_decode_batch, reference Rng), 10 layers of
    N(0,1) fp16 pages at a random page permutation, one new token per session."""
    import torch
    import oracle
    import cpp_inference_train_engine_amd as mla
    from cpp_inference_train_engine_amd.ops import latent_word, rope_word
    from cpp_inference_train_engine_amd.workloads import MLA36M as CFG3, ragged_decode_batch
    ocfg = oracle.Config.from_dict(CFG3)
    params = oracle.bits_to_f32(oracle.round_f16(oracle.model_init(ocfg, seed)))
    L, kv, rp, V, H = (ocfg.n_layers, ocfg.kv_lora_rank, ocfg.head_dim_rope, ocfg.vocab_size,
                       ocfg.n_heads)
    batch = ragged_decode_batch(B=64, n_layers=L, seed=seed)
    B, ps = batch.ctx_len.size, batch.page_size
    ctx = batch.ctx_len
    tokens = np.random.default_rng(seed).integers(0, V, size=B).astype(np.int32)
    _say(f"config3 step: B={B} cached tokens/layer={int(batch.k_len.sum())} "
         f"pages={batch.num_pages}")
    model = mla.HipModel(mla.ModelConfig.from_dict(CFG3), params, max_batch=B, page_size=ps)
    rb = mla.build_metadata(_dev(ctx), _dev(batch.q_len), _dev(batch.cu_pages),
                            _dev(batch.page_ids), ps, batch.max_pages, batch.num_pages,
                            split_pages=4, placement=placement)
    gpu_pages = [_dev(batch.pages[l].view(np.int16)).view(torch.float16) for l in range(L)]
    ws = mla.decode_workspace(rb.max_work, B, H, kv)
    logits, nxt = model.step(rb, _dev(tokens), _dev(ctx), gpu_pages, ws)
    torch.cuda.synchronize()
    info = rb.read_info()
    assert info[4] == (mla.xcd_count() if placement else 0)  # the count placed for
    # every fused merge of the step found its premises (placed metadata, items on their XCD)
    assert mla.decode_status(ws) == 0
    got_pages = np.stack([p.view(torch.int16).cpu().numpy().view(np.uint16) for p in gpu_pages])
    model.close()
    del gpu_pages
    proj = oracle.output_projection(ocfg, params)
    lw_all = latent_word(np.arange(ps)[:, None], np.arange(kv)[None, :], ps, kv, rp)
    rw_all = rope_word(np.arange(ps)[:, None], np.arange(rp)[None, :], ps, kv, rp)
    want_logits, want_lat, want_rope, got_lat, got_rope = [], [], [], [], []
    for b in range(B):
        ids = batch.page_ids[batch.cu_pages[b]:batch.cu_pages[b + 1]]
        t = np.arange(int(ctx[b]))
        pg, slot = ids[t // ps], t % ps
        dec = oracle.Decoder(ocfg, params, absorbed=True, round_cache=True, proj=proj)
        dec.latent[:, :ctx[b]] = oracle.bits_to_f32(batch.pages[:, pg[:, None], lw_all[slot]])
        dec.rope[:, :ctx[b]] = oracle.bits_to_f32(batch.pages[:, pg[:, None], rw_all[slot]])
        dec.position = int(ctx[b])
        want_logits.append(dec.decode(int(tokens[b])))
        want_lat.append(dec.latent[:, ctx[b]].copy())
        want_rope.append(dec.rope[:, ctx[b]].copy())
        p_new, s_new = ids[ctx[b] // ps], ctx[b] % ps
        got_lat.append(oracle.bits_to_f32(got_pages[:, p_new, lw_all[s_new]]))
        got_rope.append(oracle.bits_to_f32(got_pages[:, p_new, rw_all[s_new]]))
    return dict(logits=logits.cpu().numpy(), next=nxt.cpu().numpy(),
                want_logits=np.stack(want_logits), lat=np.stack(got_lat),
                want_lat=np.stack(want_lat), rope=np.stack(got_rope),
                want_rope=np.stack(want_rope))


@pytest.mark.gpu
def test_model_step_config3_full_lengths(gpu, orc):
    """The headline step (config 3) at its real lengths: every one of the 64 sessions'
    logits, appended cache rows and greedy token against the oracle's CpuDecoder."""
    _check_step(_config3_case(seed=0), "config3 (64 sessions, U[128,4096])")


@pytest.mark.gpu
def test_model_step_config3_placed(gpu, orc):
    """The same step over XCD-placed metadata, as bench.py times it: every layer's decode
    attention merges its splits inside its own launch."""
    _check_step(_config3_case(seed=0, placement=True), "config3 placed (fused merge)")


@pytest.mark.gpu
def test_model_step_tiny_matches_oracle(gpu, orc):
    """tiny-test config (H=2, kv_rank=8, rope=4): generic attention path, padded tiles."""
    r = _step_case(dict(TINY, max_sequence_length=512), B=5, max_ctx=300, seed=3, page_size=16)
    _check_step(r, "tiny")


@pytest.mark.gpu
def test_model_step_16_heads_matches_oracle(gpu, orc):
    """mla36m with 16 heads: the MFMA attention path at its largest head count, and two
    query heads per XCD in qkv_kernel's grid (head h on XCD h % 8, the append workgroup
    with heads 0 and 8), whose weight blocks g6_kernel prefetches per XCD."""
    r = _step_case(dict(MLA36M, n_heads=16, max_sequence_length=1024), B=24, max_ctx=400,
                   seed=2)
    _check_step(r, "mla36m H=16")


@pytest.mark.gpu
@pytest.mark.parametrize("B, max_ctx, seed", [(16, 700, 0), (70, 300, 1)])
def test_model_step_mla36m_matches_oracle(gpu, orc, B, max_ctx, seed):
    """mla36m (config 2/3 model): MFMA attention path; B=70 spans two 64-row chunks."""
    r = _step_case(dict(MLA36M, max_sequence_length=1024), B=B, max_ctx=max_ctx, seed=seed)
    _check_step(r, f"mla36m B={B}")


@pytest.mark.gpu
@pytest.mark.parametrize("lengths", ["config3", "short"])
def test_model_step_read_ahead_changes_no_bit(gpu, lengths):
    """The L2 read-ahead of the attention's pages during qkv_kernel (default) against the
    same placed step without it (MLA_STEP_NO_READ_AHEAD), on identical copies of the pools:
    logits, greedy tokens and every page of every layer (the appended rows included) equal
    bit for bit.  A read-ahead copy of the page being appended to would make the attention
    miss the new token.  config3: 64 sessions of 128-4096 tokens; short: 64 sessions of
    1-200 tokens, where an item's first page is often the page being appended to (the
    read-ahead must skip it)."""
    import torch
    import oracle
    import cpp_inference_train_engine_amd as mla
    from cpp_inference_train_engine_amd.workloads import MLA36M as CFG3, ragged_decode_batch
    ocfg = oracle.Config.from_dict(CFG3)
    params = oracle.bits_to_f32(oracle.round_f16(oracle.model_init(ocfg, 3)))
    batch = (ragged_decode_batch(B=64, n_layers=ocfg.n_layers, seed=3) if lengths == "config3"
             else ragged_decode_batch(B=64, n_layers=ocfg.n_layers, min_len=1, max_len=200,
                                      seed=4))
    B, ps = batch.ctx_len.size, batch.page_size
    tokens = _dev(np.random.default_rng(3).integers(0, ocfg.vocab_size, size=B).astype(np.int32))
    model = mla.HipModel(mla.ModelConfig.from_dict(CFG3), params, max_batch=B, page_size=ps)
    rb = mla.build_metadata(_dev(batch.ctx_len), _dev(batch.q_len), _dev(batch.cu_pages),
                            _dev(batch.page_ids), ps, batch.max_pages, batch.num_pages,
                            split_pages=4, placement=True)
    ws = mla.decode_workspace(rb.max_work, B, ocfg.n_heads, ocfg.kv_lora_rank)
    out = {}
    for ahead in (True, False):
        pools = [_dev(batch.pages[l].view(np.int16)).view(torch.float16)
                 for l in range(ocfg.n_layers)]
        logits, nxt = model.step(rb, tokens, _dev(batch.ctx_len), pools, ws, read_ahead=ahead)
        torch.cuda.synchronize()
        assert mla.decode_status(ws) == 0
        out[ahead] = (logits.cpu().numpy(), nxt.cpu().numpy(),
                      np.stack([p.view(torch.int16).cpu().numpy() for p in pools]))
        del pools
    model.close()
    _say(f"read-ahead vs none: max |logit diff| {np.abs(out[True][0] - out[False][0]).max():.3e}")
    assert np.array_equal(out[True][0].view(np.uint32), out[False][0].view(np.uint32))
    assert np.array_equal(out[True][1], out[False][1])
    assert np.array_equal(out[True][2], out[False][2])
