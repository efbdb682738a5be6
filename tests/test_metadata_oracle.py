"""Pins the oracle's ragged-batch metadata builder (no reference function exists).

An independent pure-Python builder written from the definitions, plus the
invariants the attention and append kernels rely on: monotone prefix sums,
every (session, page) covered by exactly one work item, slot mapping inside the
session's own pages, prefix sharing through aliased page ids.
"""
import numpy as np
import pytest


def py_metadata(ctx, q, cu_pages, page_ids, ps, max_pages, pool, split_pages, target, max_work,
                max_rows):
    B = len(ctx)
    cuq, cuk, total_pages = [0], [0], 0
    for b in range(B):
        npages = cu_pages[b + 1] - cu_pages[b]
        kl = ctx[b] + q[b]
        need = -(-kl // ps)
        ids = page_ids[cu_pages[b]:cu_pages[b + 1]]
        bad = (q[b] < 0 or ctx[b] < 0 or npages < 0 or npages > max_pages or need > npages or
               any(p < 0 or p >= pool for p in ids))
        cuq.append(cuq[-1] + q[b])
        cuk.append(cuk[-1] + kl)
        if bad or cuq[-1] > 2**31 - 1 or cuk[-1] > 2**31 - 1 or cuq[-1] > max_rows:
            return ("error", b)
        if q[b] > 0:
            total_pages += need
    split = split_pages if split_pages > 0 else max(1, -(-total_pages // target))
    ns = [(-(-(-(-(ctx[b] + q[b]) // ps)) // split) if q[b] > 0 else 0) for b in range(B)]
    cus = [0]
    for b in range(B):
        cus.append(cus[-1] + ns[b])
        if cus[-1] > max_work:
            return ("error", b)
    ws, wsp, table, slots, desc, wpages = [], [], [], [], [], []
    for b in range(B):
        ws += [b] * ns[b]
        wsp += list(range(ns[b]))
        ids = list(page_ids[cu_pages[b]:cu_pages[b + 1]])
        need = -(-(ctx[b] + q[b]) // ps)
        for sp in range(ns[b]):
            p0, p1 = sp * split, min(need, sp * split + split)
            desc.append([b, cuq[b], ctx[b] + q[b], p0, p1, ns[b], cus[b], q[b]])
            wpages.append([ids[p0 + j] if p0 + j < p1 else -1 for j in range(8)])
        table.append(ids + [-1] * (max_pages - len(ids)))
        for i in range(q[b]):
            pos = ctx[b] + i
            slots.append(ids[pos // ps] * ps + pos % ps)
    return dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, num_splits=ns, cu_splits=cus,
                work_session=ws, work_split=wsp, page_table=table, slot_mapping=slots,
                work_desc=desc, work_pages=wpages, info=[cus[-1], split, cuq[-1], cuk[-1]])


def random_batch(rng, B, ps=64, max_ctx=4096, decode=True, share_prefix=False, spare=2):
    ctx = rng.integers(0, max_ctx, B)
    q = np.ones(B, np.int64) if decode else rng.integers(0, 9, B)
    need = -(-(ctx + q) // ps)
    counts = need + rng.integers(0, spare + 1, B)
    P = int(counts.sum()) + 5
    perm = rng.permutation(P)
    ids, o = [], 0
    prefix = list(perm[:4])
    for b in range(B):
        lst = list(perm[o:o + counts[b]])
        if share_prefix and b % 2 == 0 and len(lst) >= 4:
            lst[:4] = prefix  # aliased shared-prefix pages
        ids += lst
        o += counts[b]
    cu_pages = np.concatenate([[0], np.cumsum(counts)])
    return ctx, q, cu_pages, np.array(ids), P, int(counts.max()) + 1


def run_oracle(orc, ctx, q, cu_pages, ids, ps, max_pages, P, split, target, max_work, max_rows):
    try:
        md = orc.build_metadata(ctx, q, cu_pages, ids, ps, max_pages, P, split, target, max_work)
    except ValueError as e:
        return ("error", int(str(e).split("session ")[1].rstrip(")")))
    return md


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("split", [0, 1, 3])
def test_metadata_matches_independent_builder(orc, seed, split):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 150))
    ctx, q, cu_pages, ids, P, max_pages = random_batch(rng, B, decode=seed % 2 == 0,
                                                       share_prefix=seed % 3 == 0)
    target = int(rng.integers(1, 600))
    want = py_metadata(list(ctx), list(q), list(cu_pages), list(ids), 64, max_pages, P, split,
                       target, 65535, 1 << 20)
    got = orc.build_metadata(ctx, q, cu_pages, ids, 64, max_pages, P, split, target, 65535)
    for k in ("cu_seqlens_q", "cu_seqlens_k", "num_splits", "cu_splits", "work_session",
              "work_split", "slot_mapping"):
        np.testing.assert_array_equal(got[k], np.array(want[k], np.int32), err_msg=k)
    np.testing.assert_array_equal(got["page_table"], np.array(want["page_table"], np.int32))
    np.testing.assert_array_equal(got["info"], np.array(want["info"], np.int32))
    W = want["info"][0]
    np.testing.assert_array_equal(got["work_desc"][:W], np.array(want["work_desc"], np.int32)
                                  .reshape(-1, 8))
    np.testing.assert_array_equal(got["work_pages"][:W], np.array(want["work_pages"], np.int32)
                                  .reshape(-1, 8))
    assert np.all(got["work_desc"][W:, 0] == -1)


def test_metadata_invariants(orc):
    rng = np.random.default_rng(11)
    ctx, q, cu_pages, ids, P, max_pages = random_batch(rng, 64, share_prefix=True)
    md = orc.build_metadata(ctx, q, cu_pages, ids, 64, max_pages, P, 0, 512, 65535)
    W, split, total_q, total_k = md["info"].tolist()
    assert total_q == q.sum() and total_k == (ctx + q).sum()
    assert np.all(np.diff(md["cu_seqlens_k"]) == ctx + q)
    need = -(-(ctx + q) // 64)
    assert split == max(1, -(-int(need.sum()) // 512))
    # every (session, page < need) is covered by exactly one work item
    cover = {}
    for w in range(W):
        b, sp = md["work_session"][w], md["work_split"][w]
        for p in range(sp * split, min(need[b], (sp + 1) * split)):
            cover[(b, p)] = cover.get((b, p), 0) + 1
    assert cover == {(b, p): 1 for b in range(64) for p in range(need[b])}
    # appended slot lies in the session's own page at the right offset
    for b in range(64):
        slot = md["slot_mapping"][md["cu_seqlens_q"][b]]
        assert slot // 64 == ids[cu_pages[b] + ctx[b] // 64] and slot % 64 == ctx[b] % 64


@pytest.mark.parametrize("case", ["neg_q", "short_pages", "bad_id", "too_many_pages",
                                  "max_work", "max_rows"])
def test_metadata_errors_name_first_bad_session(orc, case):
    rng = np.random.default_rng(3)
    ctx, q, cu_pages, ids, P, max_pages = random_batch(rng, 20, decode=True, spare=0)
    max_work, max_rows = 65535, 1 << 20
    ctx, q, ids = ctx.copy(), q.copy(), ids.copy()
    if case == "neg_q":
        q[7] = -1
    elif case == "short_pages":
        ctx[5] = ctx[5] + 64 * 3
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
    assert want[0] == "error"
    with pytest.raises(ValueError) as e:
        orc.build_metadata(ctx, q, cu_pages, ids, 64, max_pages, P, 1, 512, max_work, max_rows)
    assert f"session {want[1]})" in str(e.value)


def test_metadata_empty_batch(orc):
    md = orc.build_metadata(np.zeros(0), np.zeros(0), np.zeros(1), np.zeros(0), 64, 4, 10, 0,
                            16, 8)
    assert md["info"].tolist() == [0, 1, 0, 0]
