"""Chunked-prefill attention (mla_prefill_attention) against the CPU oracle.

A session with q_len > 1 appends a chunk at positions ctx .. ctx+q_len-1 and query
row i attends causally to keys [0, ctx + i]: the causal attention of the reference's
full forward (src/model/ops.cpp:109-142, Model::forward) restricted to the chunk's rows,
in CpuDecoder's absorbed form (src/infer/inference.cpp:116-153).  The oracle
(oracle.attention_paged, pinned against brute-force fp64 for q_len > 1 in
test_oracle_pinning.py) scores the same 16-bit cache and query words.  Tolerance, as for
decode: |gpu - oracle| <= 2e-3 + 1e-3*|oracle| (fp16/bf16 in, fp32 accumulation).

CPU tests pin the config-4 workload generator: lengths, page coverage, prefix aliasing.
"""
import sys

import numpy as np
import pytest

RTOL, ATOL = 1e-3, 2e-3


def _dev(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _table(batch):
    table = np.full((len(batch.ctx_len), batch.max_pages), -1, np.int32)
    for b in range(len(batch.ctx_len)):
        lst = batch.page_ids[batch.cu_pages[b]:batch.cu_pages[b + 1]]
        table[b, :len(lst)] = lst
    return table


def _oracle(orc, batch, layer=0, scale=1.0 / 8.0, threads=8):
    cu_q = np.concatenate([[0], np.cumsum(batch.q_len)]).astype(np.int32)
    return orc.attention_paged(batch.n_heads, batch.kv_rank, batch.rope_dim, batch.page_size,
                               batch.dtype, cu_q, batch.k_len.astype(np.int32), _table(batch),
                               batch.pages[layer], orc.bits_to_f32(batch.q_latent, batch.dtype),
                               orc.bits_to_f32(batch.q_rope, batch.dtype), scale, want_lse=True,
                               threads=threads)


def _run(gpu, batch, layer=0, flags=0, decode=True, scale=1.0 / 8.0):
    """decode_attention (q_len == 1 rows) + prefill_attention (q_len > 1 rows) into one out."""
    import torch
    need = (batch.k_len + batch.page_size - 1) // batch.page_size
    max_work = int(((need + 3) // 4)[batch.q_len > 0].sum())
    rb = gpu.build_metadata(_dev(batch.ctx_len), _dev(batch.q_len), _dev(batch.cu_pages),
                            _dev(batch.page_ids), batch.page_size, batch.max_pages,
                            batch.num_pages, split_pages=4, max_work=max_work,
                            max_rows=int(batch.q_len.sum()))
    tdt = torch.float16 if batch.dtype == 0 else torch.bfloat16
    pages = _dev(batch.pages[layer].view(np.int16)).view(tdt)
    ql = _dev(batch.q_latent.view(np.int16)).view(tdt)
    qr = _dev(batch.q_rope.view(np.int16)).view(tdt)
    rows, H = batch.q_latent.shape[:2]
    out = torch.full((rows, H, batch.kv_rank), float("nan"), dtype=torch.float32, device="cuda")
    lse = torch.full((rows, H), float("nan"), dtype=torch.float32, device="cuda")
    if decode:
        gpu.decode_attention(rb, pages, ql, qr, scale, kv_rank=batch.kv_rank,
                             rope_dim=batch.rope_dim, dtype=batch.dtype, out=out, lse=lse,
                             flags=flags)
    gpu.prefill_attention(rb, pages, ql, qr, scale, kv_rank=batch.kv_rank,
                          rope_dim=batch.rope_dim, max_q_len=int(batch.q_len.max()),
                          dtype=batch.dtype, out=out, lse=lse, flags=flags)
    torch.cuda.synchronize()
    rb.read_info()
    return out.cpu().numpy(), lse.cpu().numpy()


def _check(got, want, what):
    err = np.abs(got - want) - (ATOL + RTOL * np.abs(want))
    worst = np.unravel_index(np.nanargmax(np.where(np.isnan(err), np.inf, err)), err.shape)
    assert np.isfinite(got).all() and err.max() <= 0, (
        f"{what}: max excess {err.max():.3g} at {worst}: gpu {got[worst]:.6g} "
        f"oracle {want[worst]:.6g}")


# ------------------------------------------------------------------ CPU ----
def test_mixed_batch_shape_and_prefix_aliasing():
    """Config 4: 8 chunks of 512 on contexts in [0, 2048], 120 decode sessions with
    log-normal lengths capped at 16384, half of the 128 sessions aliasing one 4-page
    prefix; every other page id is used exactly once."""
    from cpp_inference_train_engine_amd.workloads import mixed_prefill_batch
    b = mixed_prefill_batch(n_layers=0)
    assert (b.q_len[:8] == 512).all() and (b.q_len[8:] == 1).all()
    assert (b.ctx_len[:8] >= 0).all() and (b.ctx_len[:8] <= 2048).all()
    assert (b.k_len[8:] >= 1).all() and (b.k_len[8:] <= 16384).all()
    lists = [b.page_ids[b.cu_pages[s]:b.cu_pages[s + 1]] for s in range(128)]
    assert all(len(l) == -(-int(k) // 64) for l, k in zip(lists, b.k_len))
    prefix = lists[[s for s in range(128) if b.ctx_len[s] >= 256][0]][:4]
    sharers = [s for s in range(128) if len(lists[s]) >= 4 and (lists[s][:4] == prefix).all()]
    assert len(sharers) == 64 and all(b.ctx_len[s] >= 256 for s in sharers)
    ids, counts = np.unique(b.page_ids, return_counts=True)
    assert (ids == np.arange(b.num_pages)).all()
    assert sorted(set(counts)) == [1, 64] and (counts == 64).sum() == 4
    # the appended slots never land in a shared page
    for s in sharers:
        assert b.ctx_len[s] // 64 >= 4


# ------------------------------------------------------------------ GPU ----
@pytest.mark.gpu
def test_prefill_config4_full_size(gpu, orc):
    """Config 4 at full size (one layer): 8 x 512-token chunks + 120 decode sessions, shared
    256-token prefix, fp16 64-token pages; both kernels into one output, every row checked."""
    from cpp_inference_train_engine_amd.workloads import mixed_prefill_batch
    batch = mixed_prefill_batch(seed=0)
    _say(f"prefill config4 rows={int(batch.q_len.sum())} keys={int(batch.k_len.sum())}")
    got, lse = _run(gpu, batch)
    want, want_lse = _oracle(orc, batch)
    _check(got, want, "out")
    np.testing.assert_allclose(lse, want_lse, rtol=1e-4, atol=1e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [0, 1])
def test_prefill_edges(gpu, orc, dtype):
    """Chunk lengths and contexts at tile and page boundaries (q_len 2..200, ctx 0..1000),
    NaN bit patterns in every slot past k_len; MFMA and generic kernels; fp16 and bf16."""
    import itertools
    from cpp_inference_train_engine_amd.ops import latent_word, rope_word
    from cpp_inference_train_engine_amd.workloads import DecodeBatch, to_bits
    qs, ctxs = [2, 3, 15, 16, 17, 63, 64, 65, 200], [0, 1, 63, 64, 100, 1000]
    pairs = list(itertools.product(qs, ctxs))[::2] + [(1, 500), (1, 64), (130, 3)]
    ctx = np.array([c for _, c in pairs], np.int32)
    q = np.array([n for n, _ in pairs], np.int32)
    k = ctx + q
    need = (k + 63) // 64 + 1  # one spare page each
    P = int(need.sum())
    rng = np.random.default_rng(dtype)
    rows = int(q.sum())
    batch = DecodeBatch(
        ctx_len=ctx, q_len=q, cu_pages=np.concatenate([[0], np.cumsum(need)]).astype(np.int32),
        page_ids=rng.permutation(P).astype(np.int32), num_pages=P, max_pages=int(need.max()),
        pages=to_bits(rng.standard_normal((1, P, 64 * 144), dtype=np.float32), dtype),
        q_latent=to_bits(rng.standard_normal((rows, 8, 128), dtype=np.float32), dtype),
        q_rope=to_bits(rng.standard_normal((rows, 8, 16), dtype=np.float32), dtype),
        page_size=64, kv_rank=128, rope_dim=16, n_heads=8, dtype=dtype)
    nan = 0x7E00 if dtype == 0 else 0x7FC0
    for b in range(len(k)):
        lst = batch.page_ids[batch.cu_pages[b]:batch.cu_pages[b + 1]]
        for t in range(int(k[b]), len(lst) * 64):
            rec = batch.pages[0, lst[t // 64]]
            rec[latent_word(t % 64, np.arange(128), 64, 128, 16)] = nan
            rec[rope_word(t % 64, np.arange(16), 64, 128, 16)] = nan
    want, want_lse = _oracle(orc, batch)
    for flags in (0, 1):
        _say(f"prefill edges dtype={dtype} flags={flags} sessions={len(k)}")
        got, lse = _run(gpu, batch, flags=flags)
        _check(got, want, f"flags={flags}")
        np.testing.assert_allclose(lse, want_lse, rtol=1e-4, atol=1e-3)


@pytest.mark.gpu
def test_prefill_generic_small_heads_and_ranks(gpu, orc):
    """tiny-test shapes (H=2, kv_rank=8, rope=4, 16-token pages): the generic kernel."""
    from cpp_inference_train_engine_amd.workloads import mixed_prefill_batch
    batch = mixed_prefill_batch(n_prefill=3, chunk=21, max_prefill_ctx=40, n_decode=4,
                                median_len=30, max_len=60, prefix_tokens=16, page_size=16,
                                n_heads=2, kv_rank=8, rope_dim=4, seed=4)
    got, lse = _run(gpu, batch, scale=0.25)
    want, want_lse = _oracle(orc, batch, scale=0.25)
    _check(got, want, "out")
    np.testing.assert_allclose(lse, want_lse, rtol=1e-4, atol=1e-3)


@pytest.mark.gpu
def test_prefill_leaves_decode_rows_alone(gpu, orc):
    """Without the decode call, rows of q_len == 1 sessions keep their contents."""
    from cpp_inference_train_engine_amd.workloads import mixed_prefill_batch
    batch = mixed_prefill_batch(n_prefill=2, chunk=40, n_decode=5, seed=2)
    got, _ = _run(gpu, batch, decode=False)
    want, _ = _oracle(orc, batch)
    dec_rows = np.concatenate([[0], np.cumsum(batch.q_len)])[2:-1]
    assert np.isnan(got[dec_rows]).all()
    _check(got[:80], want[:80], "prefill rows")


@pytest.mark.gpu
@pytest.mark.parametrize("max_pages", [2048, 2049])
def test_prefill_wide_page_table(gpu, orc, max_pages):
    """The MFMA kernel stages a session's page ids in LDS (up to 2048 pages per session);
    a wider page table (max_pages 2049) takes the generic kernel.  Same results either way."""
    import dataclasses
    from cpp_inference_train_engine_amd.workloads import mixed_prefill_batch
    batch = mixed_prefill_batch(n_prefill=2, chunk=70, max_prefill_ctx=300, n_decode=3,
                                seed=5)
    batch = dataclasses.replace(batch, max_pages=max_pages)
    _say(f"prefill wide table max_pages={max_pages}")
    got, lse = _run(gpu, batch)
    want, want_lse = _oracle(orc, batch)
    _check(got, want, f"max_pages={max_pages}")
    np.testing.assert_allclose(lse, want_lse, rtol=1e-4, atol=1e-3)
