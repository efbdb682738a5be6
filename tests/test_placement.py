"""XCD placement of the work list and the decode launch that merges its own splits.

Placement is integer work (bit-exact against the oracle's restatement, itself pinned by an
independent builder and a hand-worked case in test_metadata_oracle.py).  The fused decode
(MLA_DECODE_FUSED_MERGE over placed metadata) is fp16 in, fp32 accumulation: against the
oracle within |gpu - oracle| <= 2e-3 + 1e-3*|oracle|, and against the two-launch path
(same partials, another summation order of the merge) within 1e-5.
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


def _placed(gpu, ctx, q, cu_pages, ids, ps, max_pages, P, split, max_work, placement=True):
    import torch
    rb = gpu.build_metadata(_dev(np.asarray(ctx, np.int32)), _dev(np.asarray(q, np.int32)),
                            _dev(np.asarray(cu_pages, np.int32)),
                            _dev(np.asarray(ids if len(ids) else [0], np.int32)), ps, max_pages,
                            P, split_pages=split, max_work=max_work, max_rows=1 << 16,
                            placement=placement)
    torch.cuda.synchronize()
    return rb


def test_device_dispatch_is_round_robin_over_xcds(gpu):
    """The premise of placement: workgroup w of a launch runs on XCD w % n."""
    n = gpu.xcd_count()
    _say(f"xcd count {n}")
    assert n == 8  # MI355X: 8 XCDs, round-robin dispatch


@pytest.mark.parametrize("B, max_pages, split, seed", [
    (64, 64, 4, 0),    # config-3 shape (LDS build: B * max_pages <= 8192)
    (128, 256, 4, 1),  # config-4 decode shape (build with the page table outside LDS)
    (1, 8, 4, 2), (7, 40, 1, 3), (256, 20, 2, 4), (200, 70, 3, 5)])
def test_placed_metadata_bit_exact(gpu, orc, B, max_pages, split, seed):
    from test_metadata_oracle import random_batch
    rng = np.random.default_rng(500 + seed)
    ctx, q, cu_pages, ids, P, mp = random_batch(rng, B, decode=seed % 2 == 0,
                                                max_ctx=64 * (max_pages - 3))
    max_pages = max(max_pages, mp)
    n = gpu.xcd_count()
    max_work = gpu.placed_work_slots(ctx, q, 64, split, n) + 5
    _say(f"placed metadata B={B} max_pages={max_pages} split={split} max_work={max_work}")
    want = orc.build_metadata(ctx, q, cu_pages, ids, 64, max_pages, P, split, 512, max_work,
                              placement_xcds=n)
    rb = _placed(gpu, ctx, q, cu_pages, ids, 64, max_pages, P, split, max_work)
    assert rb.read_info() == want["info"].tolist()
    desc = rb.work_desc.cpu().numpy().reshape(-1, 8)
    occ = want["occupied"]
    np.testing.assert_array_equal(desc[:, 0] >= 0, occ)
    np.testing.assert_array_equal(desc[occ], want["work_desc"][occ])
    np.testing.assert_array_equal(rb.work_pages.cpu().numpy().reshape(-1, 8)[occ],
                                  want["work_pages"][occ])
    np.testing.assert_array_equal(rb.work_session.cpu().numpy()[occ], want["work_session"][occ])
    np.testing.assert_array_equal(rb.work_split.cpu().numpy()[occ], want["work_split"][occ])
    for k in ("cu_seqlens_q", "num_splits", "cu_splits"):
        np.testing.assert_array_equal(getattr(rb, k)[:B].cpu().numpy(), want[k][:B], err_msg=k)


def test_placed_metadata_capacity_error(gpu, orc):
    """max_work that holds the items but not the placed list: info {-1, B}, no work."""
    from test_metadata_oracle import random_batch
    rng = np.random.default_rng(9)
    ctx, q, cu_pages, ids, P, max_pages = random_batch(rng, 30)
    n = gpu.xcd_count()
    W = int((-(-(-(-(ctx + q) // 64)) // 4)).sum())
    slots = gpu.placed_work_slots(ctx, q, 64, 4, n)
    assert W < slots
    rb = _placed(gpu, ctx, q, cu_pages, ids, 64, max_pages, P, 4, slots - 1)
    with pytest.raises(gpu.MlaError):
        rb.read_info()
    assert rb.info.cpu().numpy().tolist()[:2] == [-1, 30]
    assert np.all(rb.work_desc.cpu().numpy().reshape(-1, 8)[:, 0] == -1)


def _attn(gpu, rb, batch, layer, fused, ws, lse):
    import torch
    pages = _dev(batch.pages[layer].view(np.int16)).view(torch.float16)
    ql = _dev(batch.q_latent.view(np.int16)).view(torch.float16)
    qr = _dev(batch.q_rope.view(np.int16)).view(torch.float16)
    out = gpu.decode_attention(rb, pages, ql, qr, 0.125, kv_rank=batch.kv_rank,
                               rope_dim=batch.rope_dim, lse=lse, workspace=ws, fused=fused)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check(got, want, what):
    err = np.abs(got - want) - (ATOL + RTOL * np.abs(want))
    assert err.max() <= 0, f"{what}: max excess {err.max():.3g}"


def test_fused_decode_config3_and_reuse(gpu, orc):
    """Config 3 at full size through the one-launch decode on placed metadata, every layer
    pool in turn on one workspace (the counters must come back to zero after each call),
    then a smaller batch with edge lengths on the same workspace."""
    import torch
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    from test_gpu_kernels import _oracle_decode
    batch = ragged_decode_batch(B=64, n_layers=3, seed=0)
    n = gpu.xcd_count()
    slots = gpu.placed_work_slots(batch.ctx_len, batch.q_len, 64, 4, n)
    ws = gpu.decode_workspace(slots + 64, 64, batch.n_heads, batch.kv_rank)
    rb = _placed(gpu, batch.ctx_len, batch.q_len, batch.cu_pages, batch.page_ids, 64,
                 batch.max_pages, batch.num_pages, 4, slots)
    rb0 = _placed(gpu, batch.ctx_len, batch.q_len, batch.cu_pages, batch.page_ids, 64,
                  batch.max_pages, batch.num_pages, 4, slots, placement=False)
    assert rb.read_info()[0] > 64  # split sessions present
    for layer in range(3):
        _say(f"fused decode config3 layer {layer}")
        lse = torch.zeros((64, batch.n_heads), dtype=torch.float32, device="cuda")
        got = _attn(gpu, rb, batch, layer, True, ws, lse)
        ref = _attn(gpu, rb0, batch, layer, False, ws, None)
        want, want_lse = _oracle_decode(orc, batch, layer=layer)
        _check(got, want, f"fused layer {layer}")
        np.testing.assert_allclose(lse.cpu().numpy(), want_lse, rtol=1e-4, atol=1e-3)
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)
    assert int(ws[:1024].view(torch.int32).abs().sum()) == 0  # the merge counters
    lens = [1, 2, 63, 64, 65, 127, 128, 129, 1000, 4096, 5000, 77]
    small = ragged_decode_batch(lengths=lens, seed=4, spare_pages=1)
    s_slots = gpu.placed_work_slots(small.ctx_len, small.q_len, 64, 4, n)
    rbs = _placed(gpu, small.ctx_len, small.q_len, small.cu_pages, small.page_ids, 64,
                  small.max_pages, small.num_pages, 4, s_slots)
    _say("fused decode edge lengths")
    got = _attn(gpu, rbs, small, 0, True, ws, None)
    want, _ = _oracle_decode(orc, small)
    _check(got, want, "fused edge lengths")


@pytest.mark.parametrize("n_heads", [16, 5])
def test_fused_decode_other_head_counts(gpu, orc, n_heads):
    """The MFMA page kernel serves up to 16 heads: the fused merge with two elements per
    thread (16 heads) and with an odd head count (the (m, l) blocks padded to whole lines)."""
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    from test_gpu_kernels import _oracle_decode
    batch = ragged_decode_batch(B=40, min_len=1, max_len=3000, n_heads=n_heads, seed=11)
    n = gpu.xcd_count()
    slots = gpu.placed_work_slots(batch.ctx_len, batch.q_len, 64, 4, n)
    ws = gpu.decode_workspace(slots, 40, n_heads, batch.kv_rank)
    rb = _placed(gpu, batch.ctx_len, batch.q_len, batch.cu_pages, batch.page_ids, 64,
                 batch.max_pages, batch.num_pages, 4, slots)
    _say(f"fused decode H={n_heads} items={rb.read_info()[0]}")
    got = _attn(gpu, rb, batch, 0, True, ws, None)
    want, _ = _oracle_decode(orc, batch)
    _check(got, want, f"fused H={n_heads}")


@pytest.mark.parametrize("n_xcd, B, seed", [(1, 256, 0), (1, 70, 1), (2, 256, 2), (2, 129, 3),
                                            (3, 200, 4), (3, 256, 5), (5, 256, 6), (8, 256, 7)])
def test_placed_metadata_any_xcd_count(gpu, orc, n_xcd, B, seed):
    """The placed layout for an explicit XCD count (mla_build_metadata_placed), bit-exact
    against the oracle's placement up to 256 sessions: with n = 1..3 there are more than 64
    rounds of n sessions, which the builder deals 64 rounds per pass."""
    from test_metadata_oracle import random_batch
    rng = np.random.default_rng(700 + seed)
    ctx, q, cu_pages, ids, P, mp = random_batch(rng, B, decode=seed % 2 == 0, max_ctx=2000)
    max_work = gpu.placed_work_slots(ctx, q, 64, 4, n_xcd) + 3
    _say(f"placed metadata n_xcd={n_xcd} B={B} max_work={max_work}")
    want = orc.build_metadata(ctx, q, cu_pages, ids, 64, mp, P, 4, 512, max_work,
                              placement_xcds=n_xcd)
    rb = gpu.build_metadata(_dev(np.asarray(ctx, np.int32)), _dev(np.asarray(q, np.int32)),
                            _dev(np.asarray(cu_pages, np.int32)), _dev(np.asarray(ids, np.int32)),
                            64, mp, P, split_pages=4, max_work=max_work, max_rows=1 << 16,
                            placement_xcds=n_xcd)
    assert rb.read_info() == want["info"].tolist() and want["info"][4] == n_xcd
    occ = want["occupied"]
    desc = rb.work_desc.cpu().numpy().reshape(-1, 8)
    np.testing.assert_array_equal(desc[:, 0] >= 0, occ)
    np.testing.assert_array_equal(desc[occ], want["work_desc"][occ])
    np.testing.assert_array_equal(rb.work_pages.cpu().numpy().reshape(-1, 8)[occ],
                                  want["work_pages"][occ])


def test_fused_decode_config4_as_benched(gpu, orc):
    """Config 4 exactly as bench.py's config-4 leg runs it: XCD-placed metadata for the 128
    sessions, the one-launch decode (merge inside the launch; decode sessions of up to
    16,384 tokens, i.e. up to 64 splits folded 16 at a time), then the chunked-prefill
    kernel into the same output.  Every row and its lse against the oracle."""
    import torch
    from cpp_inference_train_engine_amd.workloads import mixed_prefill_batch
    from test_prefill import _check as _check_rows, _oracle
    b = mixed_prefill_batch(seed=0)
    n = gpu.xcd_count()
    mw = gpu.placed_work_slots(b.ctx_len, b.q_len, 64, 4, n)
    rows = int(b.q_len.sum())
    rb = gpu.build_metadata(_dev(b.ctx_len), _dev(b.q_len), _dev(b.cu_pages), _dev(b.page_ids),
                            64, b.max_pages, b.num_pages, split_pages=4, max_work=mw,
                            max_rows=rows, placement=True)
    nsp = -(-((b.k_len + 63) // 64) // 4)
    _say(f"fused decode config4: max_work={mw} max splits={int(nsp.max())}")
    assert nsp[b.q_len == 1].max() > 32  # sessions past two groups of 16 splits
    pages = _dev(b.pages[0].view(np.int16)).view(torch.float16)
    ql = _dev(b.q_latent.view(np.int16)).view(torch.float16)
    qr = _dev(b.q_rope.view(np.int16)).view(torch.float16)
    out = torch.full((rows, 8, 128), float("nan"), dtype=torch.float32, device="cuda")
    lse = torch.full((rows, 8), float("nan"), dtype=torch.float32, device="cuda")
    ws = gpu.decode_workspace(mw, len(b.q_len), 8, 128)
    gpu.decode_attention(rb, pages, ql, qr, 0.125, kv_rank=128, rope_dim=16, out=out, lse=lse,
                         workspace=ws)
    gpu.prefill_attention(rb, pages, ql, qr, 0.125, kv_rank=128, rope_dim=16, max_q_len=512,
                          out=out, lse=lse)
    torch.cuda.synchronize()
    assert rb.read_info()[4] == n and rb.placed
    assert gpu.decode_status(ws) == 0
    want, want_lse = _oracle(orc, b)
    got = out.cpu().numpy()
    _check_rows(got, want, "config4 fused decode + prefill")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, rtol=1e-4, atol=1e-3)


def test_fused_decode_every_fold_group_size(gpu, orc):
    """Sessions whose split counts are 1, 2, 15, 16, 17, 32, 33 and 64 (16,384 tokens): the
    merging item folds its session's partials 16 at a time, so every group size of the fold
    (full groups and a remainder of 1) runs.  NaN in the unused slots of every last page."""
    import torch
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    from test_gpu_kernels import _oracle_decode
    lens = [100, 300, 3800, 4096, 4097, 8192, 8193, 16384, 64, 16383]
    batch = ragged_decode_batch(lengths=lens, seed=21)
    ps = 64
    for b, k in enumerate(batch.k_len):  # garbage past each session's end
        last = batch.page_ids[batch.cu_pages[b + 1] - 1]
        from cpp_inference_train_engine_amd.ops import latent_word, rope_word
        slots = np.arange(int(k) % ps or ps, ps)
        if slots.size:
            lw = latent_word(slots[:, None], np.arange(128)[None, :], ps, 128, 16)
            rw = rope_word(slots[:, None], np.arange(16)[None, :], ps, 128, 16)
            batch.pages[0, last, lw] = 0x7E00
            batch.pages[0, last, rw] = 0x7E00
    nsp = -(-((batch.k_len + 63) // 64) // 4)
    assert sorted(set(nsp.tolist())) == [1, 2, 15, 16, 17, 32, 33, 64]
    n = gpu.xcd_count()
    mw = gpu.placed_work_slots(batch.ctx_len, batch.q_len, 64, 4, n)
    rb = _placed(gpu, batch.ctx_len, batch.q_len, batch.cu_pages, batch.page_ids, 64,
                 batch.max_pages, batch.num_pages, 4, mw)
    ws = gpu.decode_workspace(mw, len(lens), 8, 128)
    _say(f"fused decode fold groups: splits {nsp.tolist()}")
    lse = torch.zeros((len(lens), 8), dtype=torch.float32, device="cuda")
    got = _attn(gpu, rb, batch, 0, True, ws, lse)
    want, want_lse = _oracle_decode(orc, batch)
    _check(got, want, "fused fold groups")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, rtol=1e-4, atol=1e-3)
    assert gpu.decode_status(ws) == 0
    assert int(ws[:1024].view(torch.int32).abs().sum()) == 0  # counters back to zero


def test_fused_flag_over_unplaced_metadata_is_flagged_not_wrong(gpu, orc):
    """MLA_DECODE_FUSED_MERGE through the C ABI over metadata in session order, and over
    metadata placed for another XCD count: the kernel does not merge, sets the session rows
    of split sessions to NaN (one-item sessions are final), leaves the partials, and raises
    MLA_DECODE_STATUS_UNPLACED; mla_decode_merge then completes every row."""
    import torch
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    from test_gpu_kernels import _oracle_decode
    batch = ragged_decode_batch(B=24, min_len=1, max_len=2500, seed=13)
    want, _ = _oracle_decode(orc, batch)
    one_item = -(-((batch.k_len + 63) // 64) // 4) == 1
    assert one_item.any() and not one_item.all()
    n = gpu.xcd_count()
    for label, kw in (("session order", {}), ("placed for 3 XCDs", {"placement_xcds": 3})):
        mw = gpu.placed_work_slots(batch.ctx_len, batch.q_len, 64, 4, 3) + 64
        rb = gpu.build_metadata(_dev(batch.ctx_len), _dev(batch.q_len), _dev(batch.cu_pages),
                                _dev(batch.page_ids), 64, batch.max_pages, batch.num_pages,
                                split_pages=4, max_work=mw, max_rows=64, **kw)
        assert not rb.placed and rb.read_info()[4] == kw.get("placement_xcds", 0) != n
        ws = gpu.decode_workspace(mw, 24, 8, 128)
        rb.placed = True  # get past the wrapper's guard to the kernel's own check
        _say(f"fused flag over unplaced metadata: {label}")
        out = torch.zeros((24, 8, 128), dtype=torch.float32, device="cuda")
        pages = _dev(batch.pages[0].view(np.int16)).view(torch.float16)
        ql = _dev(batch.q_latent.view(np.int16)).view(torch.float16)
        qr = _dev(batch.q_rope.view(np.int16)).view(torch.float16)
        gpu.decode_attention(rb, pages, ql, qr, 0.125, kv_rank=128, rope_dim=16, out=out,
                             workspace=ws, fused=True)
        torch.cuda.synchronize()
        assert gpu.decode_status(ws) == gpu.DECODE_STATUS_UNPLACED
        got = out.cpu().numpy()
        assert np.isnan(got[~one_item]).all()
        _check(got[one_item], want[one_item], f"{label}: one-item rows")
        gpu.decode_merge(rb, 8, 128, out, ws)
        torch.cuda.synchronize()
        _check(out.cpu().numpy(), want, f"{label}: after mla_decode_merge")
        assert gpu.decode_status(ws, clear=True) == gpu.DECODE_STATUS_UNPLACED
        assert gpu.decode_status(ws) == 0


def test_stale_merge_counts_are_reported(gpu, orc):
    """What a broken placement leaves behind -- a session whose items ran on several XCDs
    counts in several L2s, nobody merges it and its counter stays nonzero -- is reported as
    MLA_DECODE_STATUS_XCD.  Planted here from the host (a stale count in the workspace head),
    it stays visible after further fused calls until the head is cleared; with a clean head
    the status is 0 and the rows are the oracle's."""
    import torch
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    from test_gpu_kernels import _oracle_decode
    batch = ragged_decode_batch(B=16, min_len=300, max_len=3000, seed=17)
    n = gpu.xcd_count()
    mw = gpu.placed_work_slots(batch.ctx_len, batch.q_len, 64, 4, n)
    rb = _placed(gpu, batch.ctx_len, batch.q_len, batch.cu_pages, batch.page_ids, 64,
                 batch.max_pages, batch.num_pages, 4, mw)
    ws = gpu.decode_workspace(mw, 16, 8, 128)
    want, _ = _oracle_decode(orc, batch)
    got = _attn(gpu, rb, batch, 0, True, ws, None)
    assert gpu.decode_status(ws) == 0
    _check(got, want, "clean head")
    ns = -(-((batch.k_len + 63) // 64) // 4)
    s = int(np.argmax(ns))
    assert ns[s] > 1
    ws[:1024].view(torch.int32)[s] = 1  # a count left by an earlier call
    _say(f"fused decode over a stale count of session {s} ({int(ns[s])} splits)")
    _attn(gpu, rb, batch, 0, True, ws, None)
    assert gpu.decode_status(ws) == gpu.DECODE_STATUS_XCD
    _attn(gpu, rb, batch, 0, True, ws, None)
    assert gpu.decode_status(ws, clear=True) == gpu.DECODE_STATUS_XCD
    assert gpu.decode_status(ws) == 0
    got = _attn(gpu, rb, batch, 0, True, ws, None)
    assert gpu.decode_status(ws) == 0
    _check(got, want, "after clearing")
