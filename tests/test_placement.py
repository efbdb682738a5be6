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
