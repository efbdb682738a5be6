"""Operator interface over the C ABI for the paged, ragged MLA decode path.

Mirrors the three subsystems of the path:
  (a) ``build_metadata``   -> ``mla_build_metadata``   (GPU ragged-batch metadata)
  (b) ``append_latent``    -> ``mla_append_latent``    (paged latent/rope append)
  (c) ``decode_attention`` -> ``mla_decode_attention`` (absorbed split-K decode)
All tensors are torch CUDA (HIP) tensors; calls are stream-ordered on the
current torch stream unless ``stream`` is given.
"""
from __future__ import annotations

from dataclasses import dataclass, field

from . import (DECODE_FUSED_MERGE, DTYPE_BF16, DTYPE_F16, INFO_INTS, MAX_WORK,
               PLACE_MAX_SESSIONS, WORK_DESC_INTS, WORK_PAGES, check, lib, ptr, stream_handle)


def _torch():
    import torch
    return torch


@dataclass
class RaggedBatch:
    """Device metadata of one continuous-batching step (all int32 tensors)."""

    B: int
    page_size: int
    max_pages: int
    num_pool_pages: int
    max_work: int
    max_rows: int
    cu_seqlens_q: object
    cu_seqlens_k: object
    page_table: object
    slot_mapping: object
    num_splits: object
    cu_splits: object
    work_session: object
    work_split: object
    work_desc: object
    work_pages: object
    info: object
    placed: bool = False  # XCD-placed for this device (decode merges inside its launch)
    host_info: list = field(default_factory=list)

    def read_info(self, stream=None):
        """Synchronise and return [W, split, total_q, total_k, n_xcd placed for, 0, 0, 0];
        raises on a bad batch."""
        import numpy as np
        h = np.zeros(INFO_INTS, np.int32)
        check(lib().mla_read_metadata_info(stream_handle(stream), ptr(self.info), h.ctypes.data))
        self.host_info = h.tolist()
        return self.host_info


def xcd_count() -> int:
    """XCDs of the current device when it keeps the workgroups w with one residue w % n on one
    XCD (the premise of XCD placement), else 0.  The first call per device runs a probe
    kernel."""
    return int(lib().mla_xcd_placement_supported())


def placed_work_slots(ctx_len, q_len, page_size: int, split_pages: int, n_xcd: int) -> int:
    """Work-list slots of an XCD-placed build (host arrays of the batch's lengths): n_xcd
    times the largest item count of one XCD, as mla_build_metadata deals the sessions
    (by pages read, largest first, in rounds of n_xcd: XCDs 0..n-1, then n-1..0, ..)."""
    import numpy as np
    ctx = np.asarray(ctx_len, np.int64)
    q = np.asarray(q_len, np.int64)
    pages = np.where(q > 0, -(-(ctx + q) // page_size), 0)
    items = -(-pages // split_pages)
    order = np.lexsort((np.arange(len(pages)), -pages))
    r = np.arange(len(pages))
    xcd = np.where((r // n_xcd) % 2 == 0, r % n_xcd, n_xcd - 1 - r % n_xcd)
    cnt = np.bincount(xcd, weights=items[order], minlength=n_xcd)
    return int(n_xcd * cnt.max()) if len(pages) else 0


def build_metadata(ctx_len, q_len, cu_pages, page_ids, page_size: int, max_pages: int,
                   num_pool_pages: int, split_pages: int = 0, target_blocks: int = 1024,
                   max_work: int | None = None, max_rows: int | None = None,
                   placement: bool = False, placement_xcds: int | None = None,
                   stream=None) -> RaggedBatch:
    """(a) Build cu_seqlens, padded page tables, slot mapping and the block-to-session
    map on the GPU (one launch).  Inputs are device int32 tensors.  ``placement``: lay
    the work list out so that each session's items run on one XCD (B <= 256; max_work
    must hold ``placed_work_slots``); decode attention over it then merges the split
    partials inside its launch.  ``placement_xcds``: the placed layout for that many XCDs
    instead of this device's (mla_build_metadata_placed; no fused merge over it unless
    the count is the device's)."""
    torch = _torch()
    dev = ctx_len.device
    B = int(ctx_len.numel())
    if max_rows is None:
        max_rows = max(1, 4 * B)
    if max_work is None:
        max_work = max(1, min(MAX_WORK, target_blocks + 2 * B))
    i32 = dict(dtype=torch.int32, device=dev)
    rb = RaggedBatch(
        B=B, page_size=page_size, max_pages=max_pages, num_pool_pages=num_pool_pages,
        max_work=max_work, max_rows=max_rows,
        cu_seqlens_q=torch.empty(B + 1, **i32), cu_seqlens_k=torch.empty(B + 1, **i32),
        page_table=torch.empty(max(1, B * max_pages), **i32),
        slot_mapping=torch.empty(max_rows, **i32), num_splits=torch.empty(max(B, 1), **i32),
        cu_splits=torch.empty(B + 1, **i32), work_session=torch.empty(max_work, **i32),
        work_split=torch.empty(max_work, **i32),
        work_desc=torch.empty(max_work * WORK_DESC_INTS, **i32),
        work_pages=torch.empty(max_work * WORK_PAGES, **i32),
        info=torch.empty(INFO_INTS, **i32),
        placed=bool(placement) or (placement_xcds is not None and placement_xcds == xcd_count()))
    if placement_xcds is not None:
        fn, place = lib().mla_build_metadata_placed, int(placement_xcds)
    else:
        fn, place = lib().mla_build_metadata, int(bool(placement))
    check(fn(
        stream_handle(stream), B, ptr(ctx_len), ptr(q_len), ptr(cu_pages), ptr(page_ids),
        page_size, max_pages, num_pool_pages, split_pages, target_blocks, max_work, max_rows,
        place, ptr(rb.cu_seqlens_q), ptr(rb.cu_seqlens_k), ptr(rb.page_table),
        ptr(rb.slot_mapping), ptr(rb.num_splits), ptr(rb.cu_splits), ptr(rb.work_session),
        ptr(rb.work_split), ptr(rb.work_desc), ptr(rb.work_pages), ptr(rb.info)))
    return rb


class PagedLatentCache:
    """Device page pool: [layers, pages, page_size * (kv_rank + rope_dim)] 16-bit words.
    Each page record is latent [page_size][kv_rank] followed by rope [page_size][rope_dim]."""

    def __init__(self, n_layers: int, num_pages: int, page_size: int, kv_rank: int,
                 rope_dim: int, dtype: int = DTYPE_F16, device="cuda", storage=None):
        torch = _torch()
        self.n_layers, self.num_pages, self.page_size = n_layers, num_pages, page_size
        self.kv_rank, self.rope_dim, self.dtype = kv_rank, rope_dim, dtype
        tdt = torch.float16 if dtype == DTYPE_F16 else torch.bfloat16
        rec = page_size * (kv_rank + rope_dim)
        if storage is None:
            storage = torch.zeros((n_layers, num_pages, rec), dtype=tdt, device=device)
        assert storage.shape == (n_layers, num_pages, rec) and storage.dtype == tdt
        self.pages = storage

    def layer(self, l: int):
        return self.pages[l]

    @property
    def record_words(self) -> int:
        return self.page_size * (self.kv_rank + self.rope_dim)


def append_latent(cache: PagedLatentCache, layer: int, ckv, krope, slot_mapping,
                  stream=None) -> None:
    """(b) Round ckv [T x kv_rank] / krope [T x rope_dim] (fp32) to the cache dtype and
    write row t to flat slot slot_mapping[t] of ``layer``'s page pool."""
    T = int(ckv.shape[0])
    assert ckv.is_contiguous() and krope.is_contiguous()
    check(lib().mla_append_latent(stream_handle(stream), T, cache.kv_rank, cache.rope_dim,
                                  cache.page_size, cache.dtype, ptr(ckv), ptr(krope),
                                  ptr(slot_mapping), cache.num_pages, ptr(cache.layer(layer))))


def decode_workspace_bytes(max_work: int, max_sessions: int, n_heads: int, kv_rank: int) -> int:
    return int(lib().mla_decode_workspace_bytes(max_work, max_sessions, n_heads, kv_rank))


def decode_workspace(max_work: int, max_sessions: int, n_heads: int, kv_rank: int,
                     device="cuda"):
    """Decode workspace (head block of merge counters and status word, split partials),
    zeroed."""
    torch = _torch()
    n = max(decode_workspace_bytes(max_work, max_sessions, n_heads, kv_rank), 4)
    return torch.zeros(n, dtype=torch.uint8, device=device)


def decode_status(workspace, clear: bool = False, stream=None) -> int:
    """Synchronise and return the decode status word of ``workspace`` (OR of
    DECODE_STATUS_XCD / DECODE_STATUS_UNPLACED raised by fused calls since it was last
    cleared; 0 when every fused merge's premises held).  ``clear`` also zeroes the head."""
    import numpy as np
    h = np.zeros(1, np.int32)
    check(lib().mla_decode_status(stream_handle(stream), ptr(workspace), int(workspace.numel()),
                                  int(bool(clear)), h.ctypes.data))
    return int(h[0])


def _decode_call(fn, batch: RaggedBatch, pages, q_latent, q_rope, scale, kv_rank, rope_dim,
                 dtype, out, lse, workspace, flags, stream, fused=None):
    torch = _torch()
    rows, H = int(q_latent.shape[0]), int(q_latent.shape[1])
    if out is None:
        out = torch.zeros((rows, H, kv_rank), dtype=torch.float32, device=q_latent.device)
    if workspace is None:
        workspace = decode_workspace(batch.max_work, batch.B, H, kv_rank, q_latent.device)
    if fused is None:
        fused = batch.placed
    if fused and not batch.placed:
        raise ValueError("fused decode needs metadata placed for this device's XCDs "
                         "(build_metadata(..., placement=True))")
    if fused:
        flags |= DECODE_FUSED_MERGE
    check(getattr(lib(), fn)(
        stream_handle(stream), batch.B, H, kv_rank, rope_dim, batch.page_size, dtype,
        float(scale), ptr(batch.cu_seqlens_q), ptr(batch.page_table), batch.max_pages,
        batch.num_pool_pages, ptr(pages), ptr(q_latent), ptr(q_rope), ptr(batch.num_splits),
        ptr(batch.cu_splits), ptr(batch.work_desc), ptr(batch.work_pages), ptr(batch.info),
        batch.max_work, ptr(out), ptr(lse), ptr(workspace), int(workspace.numel()), flags))
    return out


def decode_attention(batch: RaggedBatch, pages, q_latent, q_rope, scale: float, *,
                     kv_rank: int, rope_dim: int, dtype: int = DTYPE_F16, out=None, lse=None,
                     workspace=None, flags: int = 0, stream=None, fused: bool | None = None):
    """(c) Absorbed MLA decode attention for every session with one query row.
    q_latent [rows, H, kv_rank], q_rope [rows, H, rope_dim] in the cache dtype;
    returns out [rows, H, kv_rank] fp32 (and fills lse [rows, H] if given).  ``fused``
    (default: whether the metadata is XCD-placed) merges the splits inside the decode
    launch; it needs placed metadata."""
    return _decode_call("mla_decode_attention", batch, pages, q_latent, q_rope, scale, kv_rank,
                        rope_dim, dtype, out, lse, workspace, flags, stream, fused)


def decode_partials(batch: RaggedBatch, pages, q_latent, q_rope, scale: float, *,
                    kv_rank: int, rope_dim: int, dtype: int = DTYPE_F16, out=None, lse=None,
                    workspace=None, flags: int = 0, stream=None, fused: bool = False):
    """First launch of decode_attention: final rows of one-item sessions, split partials
    of the others in ``workspace`` (pass the same workspace to ``decode_merge``); with
    ``fused`` (placed metadata) also the rows of split sessions."""
    return _decode_call("mla_decode_partials", batch, pages, q_latent, q_rope, scale, kv_rank,
                        rope_dim, dtype, out, lse, workspace, flags, stream, fused)


def decode_merge(batch: RaggedBatch, n_heads: int, kv_rank: int, out, workspace, lse=None,
                 stream=None):
    """Second launch of decode_attention: log-sum-exp merge of the split partials."""
    check(lib().mla_decode_merge(
        stream_handle(stream), batch.B, n_heads, kv_rank, ptr(batch.cu_seqlens_q),
        ptr(batch.num_splits), ptr(batch.cu_splits), ptr(batch.info), batch.max_work, ptr(out),
        ptr(lse), ptr(workspace), int(workspace.numel())))
    return out


def prefill_attention(batch: RaggedBatch, pages, q_latent, q_rope, scale: float, *,
                      kv_rank: int, rope_dim: int, max_q_len: int, dtype: int = DTYPE_F16,
                      out=None, lse=None, flags: int = 0, stream=None):
    """(c) Absorbed MLA chunked-prefill attention for every session with q_len > 1: query
    row i of a session attends causally to its keys [0, ctx + i].  The chunk's latent
    rows must already be in ``pages``.  q_latent [rows, H, kv_rank], q_rope
    [rows, H, rope_dim] in the cache dtype; returns out [rows, H, kv_rank] fp32 (rows of
    sessions with q_len <= 1 are left as they were)."""
    torch = _torch()
    rows, H = int(q_latent.shape[0]), int(q_latent.shape[1])
    if out is None:
        out = torch.zeros((rows, H, kv_rank), dtype=torch.float32, device=q_latent.device)
    check(lib().mla_prefill_attention(
        stream_handle(stream), batch.B, H, kv_rank, rope_dim, batch.page_size, dtype,
        float(scale), ptr(batch.cu_seqlens_q), ptr(batch.cu_seqlens_k), ptr(batch.page_table),
        batch.max_pages, batch.num_pool_pages, ptr(pages), ptr(q_latent), ptr(q_rope),
        ptr(batch.info), int(max_q_len), ptr(out), ptr(lse), flags))
    return out


__all__ = ["RaggedBatch", "build_metadata", "PagedLatentCache", "append_latent",
           "decode_workspace_bytes", "decode_workspace", "decode_status", "decode_attention",
           "decode_partials", "decode_merge", "prefill_attention", "DTYPE_F16", "DTYPE_BF16"]


# ---------------------------------------------------------------- page layout ----
def page_tiled(page_size: int, kv_rank: int, rope_dim: int) -> bool:
    """Page records are tiled in MFMA-operand order for these shapes (see mla_hip.h)."""
    return page_size % 16 == 0 and kv_rank % 32 == 0 and rope_dim % 8 == 0


def latent_word(slot, r, page_size: int, kv_rank: int, rope_dim: int):
    """Word index of latent column r of token `slot` inside a page record (numpy-friendly)."""
    if not page_tiled(page_size, kv_rank, rope_dim):
        return slot * kv_rank + r
    t, n, j, g, e = slot // 16, slot % 16, r // 32, (r % 32) // 8, r % 8
    return ((t * (kv_rank // 32) + j) * 4 + g) * 128 + n * 8 + e


def rope_word(slot, c, page_size: int, kv_rank: int, rope_dim: int):
    """Word index of rope column c of token `slot` inside a page record."""
    base = page_size * kv_rank
    if not page_tiled(page_size, kv_rank, rope_dim):
        return base + slot * rope_dim + c
    t, n = slot // 16, slot % 16
    return base + (t * (rope_dim // 8) + c // 8) * 128 + n * 8 + c % 8
