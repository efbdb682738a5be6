"""GPU parity of the three kernel-level entry points against the CPU oracle.

(a) metadata and (b) append are integer/byte work: bit-exact.  (c) decode
attention is fp16/bf16 in, fp32 accumulation: |gpu - oracle| <= 2e-3 + 1e-3*|oracle|
oracle = fp32 restatement of CpuDecoder's absorbed
attention (src/infer/inference.cpp:116-153) on the same 16-bit inputs.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 2e-3


def _dev(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# ------------------------------------------------------------ metadata ----
def _gpu_metadata(mla, ctx, q, cu_pages, ids, ps, max_pages, P, split, target, max_work,
                  max_rows):
    import torch
    rb = mla.build_metadata(_dev(np.asarray(ctx, np.int32)), _dev(np.asarray(q, np.int32)),
                            _dev(np.asarray(cu_pages, np.int32)),
                            _dev(np.asarray(ids if len(ids) else [0], np.int32)), ps, max_pages,
                            P, split_pages=split, target_blocks=target, max_work=max_work,
                            max_rows=max_rows)
    torch.cuda.synchronize()
    return rb


@pytest.mark.parametrize("seed", range(9))
def test_metadata_bit_exact(gpu, orc, seed):
    """Includes batches above the 4096-session LDS mirror (global-memory path)."""
    from test_metadata_oracle import random_batch
    rng = np.random.default_rng(100 + seed)
    B = [1, 7, 64, 300, 1025, 2500, 64, 130, 5000][seed]
    _say(f"metadata seed={seed} B={B}")
    ctx, q, cu_pages, ids, P, max_pages = random_batch(
        rng, B, decode=seed % 2 == 0, share_prefix=seed % 3 == 0, max_ctx=[4096, 70000][seed % 2])
    split = [0, 1, 3, 0, 2, 0, 5, 0, 0][seed]
    target = int(rng.integers(1, 2000))
    max_work, max_rows = 65535, 1 << 18
    want = orc.build_metadata(ctx, q, cu_pages, ids, 64, max_pages, P, split, target, max_work)
    rb = _gpu_metadata(gpu, ctx, q, cu_pages, ids, 64, max_pages, P, split, target, max_work,
                       max_rows)
    info = rb.read_info()
    assert info == want["info"].tolist()
    W, total_q = info[0], info[2]
    for k, n in (("cu_seqlens_q", B + 1), ("cu_seqlens_k", B + 1), ("num_splits", B),
                 ("cu_splits", B + 1), ("work_session", W), ("work_split", W),
                 ("slot_mapping", total_q)):
        np.testing.assert_array_equal(getattr(rb, k)[:n].cpu().numpy(), want[k][:n], err_msg=k)
    np.testing.assert_array_equal(rb.page_table[:B * max_pages].cpu().numpy(),
                                  want["page_table"].reshape(-1))
    desc = rb.work_desc.cpu().numpy().reshape(-1, 8)
    np.testing.assert_array_equal(desc[:W], want["work_desc"][:W])
    assert np.all(desc[W:, 0] == -1)
    np.testing.assert_array_equal(rb.work_pages.cpu().numpy().reshape(-1, 8)[:W],
                                  want["work_pages"][:W])


@pytest.mark.parametrize("B,max_pages", [(256, 64), (256, 65), (4096, 2), (4096, 5),
                                         (4097, 2)])
def test_metadata_lds_boundaries(gpu, orc, B, max_pages):
    """The build keeps the session inputs in LDS up to 4096 sessions and the padded page
    table up to 16384 entries: batches on both sides of each limit, bit-exact."""
    rng = np.random.default_rng(B + max_pages)
    ps = 64
    need = rng.integers(1, max_pages + 1, B)  # pages per session, at most max_pages
    ctx = (need - 1) * ps + rng.integers(0, ps, B)
    q = np.ones(B, np.int64)
    need = (ctx + q + ps - 1) // ps
    ctx = np.where(need > max_pages, ctx - ps, ctx)  # keep ctx + q within max_pages pages
    need = (ctx + q + ps - 1) // ps
    cu_pages = np.concatenate([[0], np.cumsum(need)])
    P = int(need.sum()) + 3
    ids = rng.permutation(P)[:int(need.sum())]
    _say(f"metadata boundary B={B} max_pages={max_pages} entries={B * max_pages}")
    want = orc.build_metadata(ctx, q, cu_pages, ids, ps, max_pages, P, 1, 512, 65535)
    rb = _gpu_metadata(gpu, ctx, q, cu_pages, ids, ps, max_pages, P, 1, 512, 65535, 1 << 16)
    assert rb.read_info() == want["info"].tolist()
    W, total_q = want["info"][0], want["info"][2]
    for k, n in (("cu_splits", B + 1), ("work_session", W), ("slot_mapping", total_q)):
        np.testing.assert_array_equal(getattr(rb, k)[:n].cpu().numpy(), want[k][:n], err_msg=k)
    np.testing.assert_array_equal(rb.page_table[:B * max_pages].cpu().numpy(),
                                  want["page_table"].reshape(-1))
    np.testing.assert_array_equal(rb.work_desc.cpu().numpy().reshape(-1, 8)[:W],
                                  want["work_desc"][:W])
    np.testing.assert_array_equal(rb.work_pages.cpu().numpy().reshape(-1, 8)[:W],
                                  want["work_pages"][:W])


@pytest.mark.parametrize("case", ["neg_q", "short_pages", "bad_id", "too_many_pages",
                                  "max_work", "max_rows"])
def test_metadata_errors_match_oracle(gpu, orc, case):
    from test_metadata_oracle import py_metadata, random_batch
    rng = np.random.default_rng(3)
    ctx, q, cu_pages, ids, P, max_pages = random_batch(rng, 20, decode=True, spare=0)
    ctx, q, ids = ctx.copy(), q.copy(), ids.copy()
    max_work, max_rows = 65535, 1 << 20
    if case == "neg_q":
        q[7] = -1
    elif case == "short_pages":
        ctx[5] += 64 * 3
    elif case == "bad_id":
        ids[cu_pages[9]] = P
    elif case == "too_many_pages":
        max_pages = int(np.diff(cu_pages).max()) - 1
    elif case == "max_work":
        max_work = 10
    elif case == "max_rows":
        max_rows = 4
    want = py_metadata(list(ctx), list(q), list(cu_pages), list(ids), 64, max_pages, P, 1, 512,
                       max_work, max_rows)
    rb = _gpu_metadata(gpu, ctx, q, cu_pages, ids, 64, max_pages, P, 1, 512, max_work, max_rows)
    with pytest.raises(gpu.MlaError) as e:
        rb.read_info()
    assert e.value.code == "invalid_argument"
    info = rb.info.cpu().numpy().tolist()
    assert info[0] == -1 and info[1] == want[1]
    assert np.all(rb.work_desc.cpu().numpy().reshape(-1, 8)[:, 0] == -1)  # no work issued


def test_metadata_empty_batch(gpu):
    rb = _gpu_metadata(gpu, [], [], [0], [], 64, 4, 10, 0, 16, 8, 8)
    assert rb.read_info() == [0, 1, 0, 0, 0, 0, 0, 0]


# -------------------------------------------------------------- append ----
@pytest.mark.parametrize("dtype", [0, 1])
def test_append_bit_exact(gpu, orc, dtype):
    import torch
    rng = np.random.default_rng(7 + dtype)
    kv, rp, ps, P, T = 128, 16, 64, 40, 300
    slots = rng.permutation(P * ps)[:T].astype(np.int32)
    ckv = rng.standard_normal((T, kv)).astype(np.float32) * rng.choice(
        [1e-8, 1e-5, 1, 300, 7e4], (T, 1)).astype(np.float32)
    kr = rng.standard_normal((T, rp)).astype(np.float32)
    ckv[0, :4] = [65519.0, 65520.0, -1e30, 2.0 ** -25]
    base = rng.integers(0, 1 << 16, (P, ps * (kv + rp)), dtype=np.uint16)
    want = base.copy()
    orc.append_paged(kv, rp, ps, dtype, ckv, kr, slots, want)
    cache = gpu.PagedLatentCache(1, P, ps, kv, rp, dtype,
                                 storage=_dev(base.view(np.int16)).view(
                                     torch.float16 if dtype == 0 else torch.bfloat16)[None])
    gpu.append_latent(cache, 0, _dev(ckv), _dev(kr), _dev(slots))
    torch.cuda.synchronize()
    got = cache.pages[0].view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)


def test_append_generic_shape_and_skips_bad_slots(gpu, orc):
    import torch
    rng = np.random.default_rng(1)
    kv, rp, ps, P, T = 8, 4, 16, 5, 20
    slots = rng.permutation(P * ps)[:T].astype(np.int32)
    slots[3] = P * ps + 7  # outside the pool: skipped, no fault
    slots[4] = -1
    ckv = rng.standard_normal((T, kv)).astype(np.float32)
    kr = rng.standard_normal((T, rp)).astype(np.float32)
    base = np.zeros((P, ps * (kv + rp)), np.uint16)
    want = base.copy()
    keep = np.ones(T, bool)
    keep[[3, 4]] = False
    orc.append_paged(kv, rp, ps, 0, ckv[keep], kr[keep], slots[keep], want)
    cache = gpu.PagedLatentCache(1, P, ps, kv, rp, 0)
    gpu.append_latent(cache, 0, _dev(ckv), _dev(kr), _dev(slots))
    torch.cuda.synchronize()
    got = cache.pages[0].view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)


# ------------------------------------------------------ decode attention ----
def _run_decode(gpu, batch, layer=0, split=0, target=1024, flags=0, want_lse=True,
                scale=1.0 / 8.0):
    import torch
    rb = gpu.build_metadata(_dev(batch.ctx_len), _dev(batch.q_len), _dev(batch.cu_pages),
                            _dev(batch.page_ids), batch.page_size, batch.max_pages,
                            batch.num_pages, split_pages=split, target_blocks=target)
    tdt = torch.float16 if batch.dtype == 0 else torch.bfloat16
    pages = _dev(batch.pages[layer].view(np.int16)).view(tdt)
    ql = _dev(batch.q_latent.view(np.int16)).view(tdt)
    qr = _dev(batch.q_rope.view(np.int16)).view(tdt)
    B, H = batch.q_latent.shape[:2]
    lse = torch.zeros((B, H), dtype=torch.float32, device="cuda") if want_lse else None
    out = gpu.decode_attention(rb, pages, ql, qr, scale, kv_rank=batch.kv_rank,
                               rope_dim=batch.rope_dim, dtype=batch.dtype, lse=lse, flags=flags)
    torch.cuda.synchronize()
    info = rb.read_info()
    return out.cpu().numpy(), (lse.cpu().numpy() if want_lse else None), info


def _oracle_decode(orc, batch, layer=0, scale=1.0 / 8.0):
    k_len = batch.k_len.astype(np.int32)
    table = np.full((len(k_len), batch.max_pages), -1, np.int32)
    for b in range(len(k_len)):
        lst = batch.page_ids[batch.cu_pages[b]:batch.cu_pages[b + 1]]
        table[b, :len(lst)] = lst
    cu_q = np.arange(len(k_len) + 1, dtype=np.int32)
    ql = orc.bits_to_f32(batch.q_latent, batch.dtype)
    qr = orc.bits_to_f32(batch.q_rope, batch.dtype)
    return orc.attention_paged(batch.n_heads, batch.kv_rank, batch.rope_dim, batch.page_size,
                               batch.dtype, cu_q, k_len, table, batch.pages[layer], ql, qr, scale,
                               want_lse=True)


def _check(got, want, what):
    err = np.abs(got - want) - (ATOL + RTOL * np.abs(want))
    worst = np.unravel_index(np.argmax(err), err.shape)
    assert err.max() <= 0, (f"{what}: max excess {err.max():.3g} at {worst}: "
                            f"gpu {got[worst]:.6g} oracle {want[worst]:.6g}")


@pytest.mark.parametrize("flags", [0, 1], ids=["mfma", "generic"])
def test_decode_config3_full_size(gpu, orc, flags):
    """Config 3 at full size: 64 sessions, len U[128,4096], fp16 64-token pages in a random
    permutation, N(0,1) contents (one layer)."""
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    batch = ragged_decode_batch(seed=0)
    _say(f"decode config3 flags={flags} tokens={int(batch.k_len.sum())}")
    got, lse, info = _run_decode(gpu, batch, flags=flags)
    want, want_lse = _oracle_decode(orc, batch)
    _check(got, want, "out")
    np.testing.assert_allclose(lse, want_lse, rtol=1e-4, atol=1e-3)
    assert info[0] > 64  # split-K actually exercised


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("split", [1, 2, 1000])
def test_decode_edge_lengths(gpu, orc, dtype, split):
    """Lengths at page boundaries (1, 63, 64, 65, 128, 129) and long sessions; one split per
    page, two pages, and one split per session; fp16 and bf16."""
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    lens = [1, 2, 63, 64, 65, 127, 128, 129, 1000, 4096, 5000, 77]
    batch = ragged_decode_batch(lengths=lens, dtype=dtype, seed=3 + dtype, spare_pages=1)
    _say(f"decode edges dtype={dtype} split={split}")
    for flags in (0, 1):
        got, lse, _ = _run_decode(gpu, batch, split=split, flags=flags)
        want, want_lse = _oracle_decode(orc, batch)
        _check(got, want, f"out flags={flags}")
        np.testing.assert_allclose(lse, want_lse, rtol=1e-4, atol=1e-3)


def test_decode_generic_small_heads_and_ranks(gpu, orc):
    """tiny-test-like shapes (H=2, kv_rank=8, rope=4, 16-token pages) use the generic kernel."""
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    batch = ragged_decode_batch(B=9, min_len=1, max_len=200, page_size=16, n_heads=2, kv_rank=8,
                                rope_dim=4, seed=5)
    got, lse, _ = _run_decode(gpu, batch, split=2)
    want, want_lse = _oracle_decode(orc, batch)
    _check(got, want, "out")


def test_decode_skips_prefill_rows_and_tolerates_garbage_slots(gpu, orc):
    """Unwritten slots past k_len hold NaN bit patterns; sessions with q_len != 1 are left
    untouched by the decode kernel."""
    import torch
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    from cpp_inference_train_engine_amd.ops import latent_word, rope_word
    batch = ragged_decode_batch(lengths=[70, 5, 200, 64], seed=8)
    # fill every slot beyond k_len with fp16 NaN
    for b, L in enumerate(batch.k_len):
        lst = batch.page_ids[batch.cu_pages[b]:batch.cu_pages[b + 1]]
        for t in range(L, len(lst) * 64):
            rec = batch.pages[0, lst[t // 64]]
            rec[latent_word(t % 64, np.arange(128), 64, 128, 16)] = 0x7E00
            rec[rope_word(t % 64, np.arange(16), 64, 128, 16)] = 0x7E00
    for flags in (0, 1):
        got, _, _ = _run_decode(gpu, batch, split=1, flags=flags)
        want, _ = _oracle_decode(orc, batch)
        assert np.isfinite(got).all()
        _check(got, want, f"flags={flags}")
    # a batch where session 1 is a 3-token prefill: its rows stay zero
    batch.q_len = np.array([1, 3, 1, 1], np.int32)
    batch.ctx_len = (batch.k_len - batch.q_len).astype(np.int32)
    q = np.zeros((6, 8, 128), np.uint16)
    q[[0, 4, 5]] = batch.q_latent[[0, 2, 3]]
    batch.q_latent = q
    qr = np.zeros((6, 8, 16), np.uint16)
    qr[[0, 4, 5]] = batch.q_rope[[0, 2, 3]]
    batch.q_rope = qr
    got, _, _ = _run_decode(gpu, batch, split=1, want_lse=False)
    assert np.all(got[1:4] == 0)
    assert np.abs(got[[0, 4, 5]]).sum() > 0


def test_decode_workspace_reuse_across_calls(gpu, orc):
    """One workspace serves consecutive calls with different batches, layers and split
    sizes (stale partials of an earlier call never leak into a later one)."""
    import torch
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    ws = gpu.decode_workspace(4096, 64, 8, 128)
    for seed, split, n in [(11, 1, 64), (12, 3, 20), (13, 0, 64), (11, 2, 64)]:
        batch = ragged_decode_batch(B=n, max_len=3000, seed=seed, n_layers=2)
        for layer in (0, 1):
            rb = gpu.build_metadata(_dev(batch.ctx_len), _dev(batch.q_len), _dev(batch.cu_pages),
                                    _dev(batch.page_ids), 64, batch.max_pages, batch.num_pages,
                                    split_pages=split, target_blocks=300, max_work=4096)
            pages = _dev(batch.pages[layer].view(np.int16)).view(torch.float16)
            ql = _dev(batch.q_latent.view(np.int16)).view(torch.float16)
            qr = _dev(batch.q_rope.view(np.int16)).view(torch.float16)
            out = gpu.decode_attention(rb, pages, ql, qr, 0.125, kv_rank=128, rope_dim=16,
                                       workspace=ws)
            torch.cuda.synchronize()
            want, _ = _oracle_decode(orc, batch, layer=layer)
            _check(out.cpu().numpy(), want, f"seed={seed} split={split} layer={layer}")


def test_decode_split_merge_repeated_calls_and_graph_replays(gpu, orc):
    """Production split (MLA_DECODE_SPLIT_PAGES pages per work item, one wave per page):
    repeated eager calls on alternating layers and HIP-graph replays (with eager work in
    between) share one workspace and must all match the oracle."""
    import torch
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    batch = ragged_decode_batch(B=64, n_layers=2, seed=5)
    _say(f"split merge: tokens={int(batch.k_len.sum())}")
    B, H = batch.q_latent.shape[:2]
    rb = gpu.build_metadata(_dev(batch.ctx_len), _dev(batch.q_len), _dev(batch.cu_pages),
                            _dev(batch.page_ids), 64, batch.max_pages, batch.num_pages,
                            split_pages=4, max_work=1024)
    info = rb.read_info()
    assert info[1] == 4 and info[0] > 2 * B
    pages = _dev(batch.pages.view(np.int16)).view(torch.float16)
    ql = _dev(batch.q_latent.view(np.int16)).view(torch.float16)
    qr = _dev(batch.q_rope.view(np.int16)).view(torch.float16)
    want = [_oracle_decode(orc, batch, layer=l)[0] for l in range(2)]
    ws = gpu.decode_workspace(1024, B, H, 128)
    out = torch.zeros((B, H, 128), dtype=torch.float32, device="cuda")
    for call in range(4):
        out.fill_(float("nan"))
        gpu.decode_attention(rb, pages[call % 2], ql, qr, 0.125, kv_rank=128, rope_dim=16,
                             out=out, workspace=ws)
        torch.cuda.synchronize()
        _check(out.cpu().numpy(), want[call % 2], f"eager call {call}")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            gpu.decode_attention(rb, pages[1], ql, qr, 0.125, kv_rank=128, rope_dim=16,
                                 out=out, workspace=ws)
    torch.cuda.synchronize()
    for rep in range(4):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        _check(out.cpu().numpy(), want[1], f"graph replay {rep}")
        gpu.decode_attention(rb, pages[0], ql, qr, 0.125, kv_rank=128, rope_dim=16, out=out,
                             workspace=ws)
        torch.cuda.synchronize()
        _check(out.cpu().numpy(), want[0], f"eager call after replay {rep}")


@pytest.mark.parametrize("flags", [0, 1], ids=["mfma", "generic"])
def test_decode_partials_then_merge_equals_attention(gpu, orc, flags):
    """mla_decode_partials + mla_decode_merge are the two launches of mla_decode_attention:
    bit-identical output and lse, and the oracle bar."""
    import torch
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    batch = ragged_decode_batch(B=40, seed=9)
    _say(f"partials+merge flags={flags}")
    B, H = batch.q_latent.shape[:2]
    rb = gpu.build_metadata(_dev(batch.ctx_len), _dev(batch.q_len), _dev(batch.cu_pages),
                            _dev(batch.page_ids), 64, batch.max_pages, batch.num_pages,
                            split_pages=4)
    pages = _dev(batch.pages[0].view(np.int16)).view(torch.float16)
    ql = _dev(batch.q_latent.view(np.int16)).view(torch.float16)
    qr = _dev(batch.q_rope.view(np.int16)).view(torch.float16)
    lse_a = torch.zeros((B, H), dtype=torch.float32, device="cuda")
    lse_b = torch.zeros((B, H), dtype=torch.float32, device="cuda")
    ref = gpu.decode_attention(rb, pages, ql, qr, 0.125, kv_rank=128, rope_dim=16, lse=lse_a,
                               flags=flags)
    ws = gpu.decode_workspace(rb.max_work, B, H, 128)
    out = torch.full((B, H, 128), float("nan"), dtype=torch.float32, device="cuda")
    gpu.decode_partials(rb, pages, ql, qr, 0.125, kv_rank=128, rope_dim=16, out=out,
                        lse=lse_b, workspace=ws, flags=flags)
    gpu.decode_merge(rb, H, 128, out, ws, lse=lse_b)
    torch.cuda.synchronize()
    assert torch.equal(out, ref) and torch.equal(lse_a, lse_b)
    want, _ = _oracle_decode(orc, batch)
    _check(out.cpu().numpy(), want, f"flags={flags}")


# --------------------------------------------- DeepSeek-like shape (config 5) ----
def _wide_batch(lengths, dtype, seed):
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    return ragged_decode_batch(lengths=lengths, n_heads=128, kv_rank=512, rope_dim=64,
                               dtype=dtype, seed=seed, spare_pages=1)


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("split", [2, 1000])
def test_decode_wide_shape_edges(gpu, orc, dtype, split):
    """H=128, kv_rank=512, rope=64 (config 5's latent shape): lengths at page boundaries,
    NaN bit patterns past every session's end, split partials and single items."""
    from cpp_inference_train_engine_amd.ops import latent_word, rope_word
    batch = _wide_batch([1, 2, 63, 64, 65, 130, 700, 1500], dtype, seed=20 + dtype)
    nan = 0x7E00 if dtype == 0 else 0x7FC0
    for b, L in enumerate(batch.k_len):
        lst = batch.page_ids[batch.cu_pages[b]:batch.cu_pages[b + 1]]
        for t in range(int(L), len(lst) * 64):
            rec = batch.pages[0, lst[t // 64]]
            rec[latent_word(t % 64, np.arange(512), 64, 512, 64)] = nan
            rec[rope_word(t % 64, np.arange(64), 64, 512, 64)] = nan
    _say(f"decode wide dtype={dtype} split={split}")
    scale = 1.0 / np.sqrt(192.0)
    want, want_lse = _oracle_decode(orc, batch, scale=scale)
    got, lse, _ = _run_decode(gpu, batch, split=split, scale=scale)
    _check(got, want, "out")
    np.testing.assert_allclose(lse, want_lse, rtol=1e-4, atol=1e-3)


def test_decode_config5_full_size(gpu, orc):
    """Config 5 at full size and at the split bench.py times (128 pages per work item):
    256 sessions, len U[8192, 32768] (reference Rng, seed 0), bf16 64-token pages in a
    random permutation, N(0,1) cache and queries drawn on the GPU (torch generator, seed 0).
    25 sessions spread over the length range (every 11th by length from the shortest, plus
    the longest) are read back and checked against the oracle; every output is finite."""
    import torch
    from cpp_inference_train_engine_amd.workloads import deepseek_decode_shape
    shape = deepseek_decode_shape(seed=0)
    _say(f"decode config5 tokens={int(shape.k_len.sum())} pages={shape.num_pages}")
    gen = torch.Generator(device="cuda").manual_seed(0)
    rec = 64 * 576
    pages = torch.randn((shape.num_pages, rec), generator=gen, device="cuda").to(torch.bfloat16)
    B = len(shape.k_len)
    ql = torch.randn((B, 128, 512), generator=gen, device="cuda").to(torch.bfloat16)
    qr = torch.randn((B, 128, 64), generator=gen, device="cuda").to(torch.bfloat16)
    need = (shape.k_len + 63) // 64
    split = 128
    max_work = int(((need + split - 1) // split).sum())
    rb = gpu.build_metadata(_dev(shape.ctx_len), _dev(shape.q_len), _dev(shape.cu_pages),
                            _dev(shape.page_ids), 64, shape.max_pages, shape.num_pages,
                            split_pages=split, max_work=max_work)
    scale = 1.0 / np.sqrt(192.0)
    out = gpu.decode_attention(rb, pages, ql, qr, scale, kv_rank=512, rope_dim=64,
                               dtype=gpu.DTYPE_BF16)
    torch.cuda.synchronize()
    rb.read_info()
    assert torch.isfinite(out).all()
    order = np.argsort(shape.k_len)
    picks = sorted(set(int(order[i]) for i in list(range(0, 256, 11)) + [255]))
    # One oracle call over the picked sessions (threads work on sessions in parallel):
    # their pages gathered into a compact pool, page table rows renumbered.
    lists = [shape.page_ids[shape.cu_pages[b]:shape.cu_pages[b + 1]] for b in picks]
    flat = np.concatenate(lists).astype(np.int64)
    sub = pages[torch.from_numpy(flat).cuda()].view(torch.int16).cpu().numpy().view(np.uint16)
    table = np.full((len(picks), max(len(x) for x in lists)), -1, np.int32)
    off = 0
    for i, x in enumerate(lists):
        table[i, :len(x)] = np.arange(off, off + len(x), dtype=np.int32)
        off += len(x)
    sel = torch.tensor(picks, device="cuda")
    bits = lambda t: t[sel].view(torch.int16).cpu().numpy().view(np.uint16)
    want = orc.attention_paged(128, 512, 64, 64, 1, np.arange(len(picks) + 1, dtype=np.int32),
                               shape.k_len[picks].astype(np.int32), table, sub,
                               orc.bits_to_f32(bits(ql), 1), orc.bits_to_f32(bits(qr), 1),
                               scale, threads=16)
    got = out[sel].cpu().numpy()
    for i, b in enumerate(picks):
        _check(got[i:i + 1], want[i:i + 1], f"session {b} (len {int(shape.k_len[b])})")
