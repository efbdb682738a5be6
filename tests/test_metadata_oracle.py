"""Pins the oracle's ragged-batch metadata builder (no reference function exists).

An independent pure-Python builder written from the definitions, plus the
invariants the attention and append kernels rely on: monotone prefix sums,
every (session, page) covered by exactly one work item, slot mapping inside the
session's own pages, prefix sharing through aliased page ids.
"""
import numpy as np
import pytest


def py_placement(pages, ns, n):
    """XCD placement restated as a deal: sessions by (pages desc, index asc) are dealt
    along the cycle 0, 1, .., n-1, n-1, .., 1, 0 of XCDs.  Returns {session: (xcd, first)}
    and the per-XCD item counts."""
    import itertools
    deal = itertools.cycle(list(range(n)) + list(range(n - 1, -1, -1)))
    items = [0] * n
    where = {}
    for b in sorted(range(len(pages)), key=lambda b: (-pages[b], b)):
        x = next(deal)
        where[b] = (x, items[x])
        items[x] += ns[b]
    return where, items


def py_metadata(ctx, q, cu_pages, page_ids, ps, max_pages, pool, split_pages, target, max_work,
                max_rows, n_xcd=0):
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
    if n_xcd:
        pages = [-(-(ctx[b] + q[b]) // ps) if q[b] > 0 else 0 for b in range(B)]
        where, items = py_placement(pages, ns, n_xcd)
        if n_xcd * max(items) > max_work:
            return ("error", B)
    ws, wsp, table, slots, desc, wpages, slot_of = [], [], [], [], [], [], []
    for b in range(B):
        ws += [b] * ns[b]
        wsp += list(range(ns[b]))
        ids = list(page_ids[cu_pages[b]:cu_pages[b + 1]])
        need = -(-(ctx[b] + q[b]) // ps)
        for sp in range(ns[b]):
            p0, p1 = sp * split, min(need, sp * split + split)
            desc.append([b, cuq[b], ctx[b] + q[b], p0, p1, ns[b], cus[b] + sp, q[b]])
            wpages.append([ids[p0 + j] if p0 + j < p1 else -1 for j in range(8)])
            slot_of.append(where[b][0] + n_xcd * (where[b][1] + sp) if n_xcd else len(slot_of))
        table.append(ids + [-1] * (max_pages - len(ids)))
        for i in range(q[b]):
            pos = ctx[b] + i
            slots.append(ids[pos // ps] * ps + pos % ps)
    return dict(cu_seqlens_q=cuq, cu_seqlens_k=cuk, num_splits=ns, cu_splits=cus,
                work_session=ws, work_split=wsp, page_table=table, slot_mapping=slots,
                work_desc=desc, work_pages=wpages,
                info=[cus[-1], split, cuq[-1], cuk[-1], n_xcd, 0, 0, 0],
                slot_of=slot_of)


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
    W, split, total_q, total_k, placed_for, *rest = md["info"].tolist()
    assert placed_for == 0 and rest == [0, 0, 0]
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
    assert md["info"].tolist() == [0, 1, 0, 0, 0, 0, 0, 0]


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("n_xcd", [1, 3, 8])
def test_placed_metadata_matches_independent_builder(orc, seed, n_xcd):
    rng = np.random.default_rng(100 + seed)
    B = int(rng.integers(1, 200))
    ctx, q, cu_pages, ids, P, max_pages = random_batch(rng, B, decode=seed % 2 == 0,
                                                       share_prefix=seed % 3 == 0)
    split = [1, 3, 4][seed % 3]
    want = py_metadata(list(ctx), list(q), list(cu_pages), list(ids), 64, max_pages, P, split,
                       512, 65535, 1 << 20, n_xcd)
    got = orc.build_metadata(ctx, q, cu_pages, ids, 64, max_pages, P, split, 512, 65535,
                             placement_xcds=n_xcd)
    for k in ("cu_seqlens_q", "cu_seqlens_k", "num_splits", "cu_splits", "slot_mapping", "info"):
        np.testing.assert_array_equal(got[k], np.array(want[k], np.int32), err_msg=k)
    slots = np.array(want["slot_of"], np.int64)
    occupied = np.zeros(65535, bool)
    occupied[slots] = True
    np.testing.assert_array_equal(got["occupied"], occupied)
    np.testing.assert_array_equal(got["work_desc"][slots],
                                  np.array(want["work_desc"], np.int32).reshape(-1, 8))
    np.testing.assert_array_equal(got["work_pages"][slots],
                                  np.array(want["work_pages"], np.int32).reshape(-1, 8))
    np.testing.assert_array_equal(got["work_session"][slots], want["work_session"])
    np.testing.assert_array_equal(got["work_split"][slots], want["work_split"])


def test_placement_known_answer(orc):
    # 4 sessions reading 5, 3, 3 and 1 pages, 2 pages per item, 2 XCDs, worked by hand:
    # ranks 0-3 are sessions 0-3; round 0 deals XCDs 0, 1 and round 1 XCDs 1, 0, so
    # session 0 -> XCD 0, 1 -> XCD 1, 2 -> XCD 1, 3 -> XCD 0 (pages 6 | 6);
    # items 3, 2, 2, 1; XCD 0 holds s0 items 0-2 then s3, XCD 1 s1 items 0-1 then s2.
    ctx = np.array([5 * 64 - 1, 3 * 64 - 1, 3 * 64 - 1, 0])
    q = np.ones(4, np.int64)
    cu_pages = np.array([0, 5, 8, 11, 12])
    ids = np.arange(12)
    md = orc.build_metadata(ctx, q, cu_pages, ids, 64, 5, 12, 2, 512, 10, placement_xcds=2)
    sess = [int(md["work_desc"][w, 0]) for w in range(10)]
    split = [int(md["work_split"][w]) if sess[w] >= 0 else -1 for w in range(10)]
    assert sess == [0, 1, 0, 1, 0, 2, 3, 2, -1, -1]
    assert split == [0, 0, 1, 1, 2, 0, 0, 1, -1, -1]
    # field 6: the partial slot cu_splits[session] + split (cu_splits = 0, 3, 5, 7)
    assert [int(md["work_desc"][w, 6]) for w in range(8)] == [0, 3, 1, 4, 2, 5, 7, 6]
    # 2 sessions of 3 and 1 items on 2 XCDs need 2 x 3 slots: max_work 5 holds the 4 items
    # but not the placed list, an error naming session B
    with pytest.raises(ValueError, match="session 2"):
        orc.build_metadata(ctx[[0, 3]], q[:2], np.array([0, 5, 6]), ids[:6], 64, 5, 12, 2, 512,
                           5, placement_xcds=2)
    md = orc.build_metadata(ctx[[0, 3]], q[:2], np.array([0, 5, 6]), ids[:6], 64, 5, 12, 2, 512,
                            6, placement_xcds=2)
    assert md["work_desc"][:, 0].tolist() == [0, 1, 0, -1, 0, -1]


def test_placement_invariants(orc):
    rng = np.random.default_rng(7)
    B, n = 120, 8
    ctx = np.minimum(rng.lognormal(np.log(2048), 1.0, B), 16384).astype(np.int64)
    ctx, q, cu_pages, ids, P, max_pages = random_batch(rng, B)
    md = orc.build_metadata(ctx, q, cu_pages, ids, 64, max_pages, P, 4, 512, 65535,
                            placement_xcds=n)
    pages = -(-(ctx + q) // 64)
    occ = np.nonzero(md["occupied"])[0]
    assert occ.size == md["info"][0]
    seen = {}
    for w in occ:
        b, sp = int(md["work_session"][w]), int(md["work_split"][w])
        seen.setdefault(b, []).append((sp, int(w)))
        assert md["work_desc"][w, 6] == md["cu_splits"][b] + sp
    load = np.zeros(n, np.int64)
    for b, lst in seen.items():
        lst.sort()
        assert [sp for sp, _ in lst] == list(range(md["num_splits"][b]))
        xs = {w % n for _, w in lst}
        assert len(xs) == 1  # one XCD per session
        ks = [w // n for _, w in lst]
        assert ks == list(range(ks[0], ks[0] + len(ks)))  # consecutive slots of that XCD
        load[xs.pop()] += pages[b]
    # one session per XCD per round, sessions in descending order: no XCD exceeds another
    # by more than the largest session's pages
    assert load.max() - load.min() <= pages.max()
    # empty slots only past each XCD's items
    per = np.bincount(occ % n, minlength=n)
    assert all(not md["occupied"][x + n * k] for x in range(n) for k in range(per[x], per.max()))
