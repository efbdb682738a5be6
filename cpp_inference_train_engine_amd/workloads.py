"""Synthetic ragged decode batches of the benchmark configurations.

Session lengths and the physical page permutation follow the reference's Rng
(SplitMix64, include/mini_mla/rng.hpp:9-28: ``bounded`` with rejection, Fisher-
Yates shuffle), so the batch shape for a seed is the same on every host.  The
bulk cache/query contents are N(0, 1) from numpy's PCG64 (seeded) and rounded
once to the 16-bit cache dtype; both the GPU and any CPU checker consume the
same rounded bits.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

M64 = (1 << 64) - 1


class SplitMix64:
    """Integer part of the reference Rng (rng.hpp:11-28)."""

    def __init__(self, seed: int):
        self.state = seed & M64

    def next(self) -> int:
        self.state = (self.state + 0x9E3779B97F4A7C15) & M64
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> 31)

    def bounded(self, bound: int) -> int:
        if bound == 0:
            return 0
        threshold = ((1 << 64) - bound) % bound
        while True:
            r = self.next()
            if r >= threshold:
                return r % bound


def to_bits(x: np.ndarray, dtype: int) -> np.ndarray:
    """Round fp32 to 16-bit words (RNE) of dtype 0 = fp16, 1 = bf16."""
    x = np.ascontiguousarray(x, np.float32)
    if dtype == 0:
        return x.astype(np.float16).view(np.uint16)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r[nan] = ((x.view(np.uint32)[nan] >> 16) | 0x40).astype(np.uint16)
    return r


@dataclass
class DecodeBatch:
    """One ragged step: session b has ctx_len[b] cached tokens and appends q_len[b]
    (1 for a decode session, a chunk for a prefill session); query rows are packed in
    session order (rows = q_len.sum())."""

    ctx_len: np.ndarray   # int32 [B] tokens already cached
    q_len: np.ndarray     # int32 [B]
    cu_pages: np.ndarray  # int32 [B+1]
    page_ids: np.ndarray  # int32 [sum pages]
    num_pages: int        # pool size
    max_pages: int
    pages: np.ndarray     # uint16 [L, num_pages, page_size*(kv+rope)]
    q_latent: np.ndarray  # uint16 [rows, H, kv]
    q_rope: np.ndarray    # uint16 [rows, H, rope]
    page_size: int
    kv_rank: int
    rope_dim: int
    n_heads: int
    dtype: int

    @property
    def k_len(self) -> np.ndarray:
        return self.ctx_len + self.q_len

    def cache_bytes_per_layer(self) -> int:
        """Algorithmic bytes one decode-attention launch must read (one layer)."""
        return int(self.k_len.sum()) * (self.kv_rank + self.rope_dim) * 2


def ragged_decode_batch(B=64, min_len=128, max_len=4096, page_size=64, n_heads=8, kv_rank=128,
                        rope_dim=16, n_layers=1, dtype=0, seed=0, spare_pages=0,
                        lengths=None, q_rows=None) -> DecodeBatch:
    """Config-3-style batch: context lengths (after the append) uniform in
    [min_len, max_len], pages of ``page_size`` tokens at a random permutation of the
    pool, N(0,1) cache and query contents."""
    rng = SplitMix64(seed)
    if lengths is None:
        k_len = np.array([min_len + rng.bounded(max_len - min_len + 1) for _ in range(B)],
                         np.int64)
    else:
        k_len = np.asarray(lengths, np.int64)
        B = k_len.size
    need = (k_len + page_size - 1) // page_size
    counts = need + spare_pages
    P = int(counts.sum())
    perm = list(range(P))
    for i in range(P - 1, 0, -1):  # Fisher-Yates with the reference Rng
        j = rng.bounded(i + 1)
        perm[i], perm[j] = perm[j], perm[i]
    page_ids = np.array(perm, np.int32)
    cu_pages = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    gen = np.random.default_rng(seed)
    rec = page_size * (kv_rank + rope_dim)
    pages = np.empty((n_layers, P, rec), np.uint16)
    for l in range(n_layers):
        pages[l] = to_bits(gen.standard_normal((P, rec), dtype=np.float32), dtype)
    rows = B if q_rows is None else q_rows
    q_latent = to_bits(gen.standard_normal((rows, n_heads, kv_rank), dtype=np.float32), dtype)
    q_rope = to_bits(gen.standard_normal((rows, n_heads, rope_dim), dtype=np.float32), dtype)
    return DecodeBatch(ctx_len=(k_len - 1).astype(np.int32), q_len=np.ones(B, np.int32),
                       cu_pages=cu_pages, page_ids=page_ids, num_pages=P,
                       max_pages=int(counts.max()), pages=pages, q_latent=q_latent,
                       q_rope=q_rope, page_size=page_size, kv_rank=kv_rank, rope_dim=rope_dim,
                       n_heads=n_heads, dtype=dtype)


def mixed_prefill_batch(n_prefill=8, chunk=512, max_prefill_ctx=2048, n_decode=120,
                        median_len=2048, sigma=1.0, max_len=16384, prefix_tokens=256,
                        n_share=None, page_size=64, n_heads=8, kv_rank=128, rope_dim=16,
                        n_layers=1, dtype=0, seed=0) -> DecodeBatch:
    """Config-4-style mixed batch: ``n_prefill`` chunks of ``chunk`` tokens appended
    (causal within the chunk) to contexts uniform in [0, max_prefill_ctx], then
    ``n_decode`` decode sessions whose lengths (after the append) are log-normal with
    median ``median_len`` and shape ``sigma``, capped at ``max_len``.  Half of the
    sessions (``n_share``) share the first ``prefix_tokens`` tokens through aliased
    page ids: the first sessions, in order, whose cached context covers the whole
    prefix (a session never appends into a shared page).  Page ids are a Fisher-Yates
    permutation of the pool (reference Rng); contents N(0, 1) rounded once."""
    rng = SplitMix64(seed)
    gen = np.random.default_rng(seed)
    B = n_prefill + n_decode
    ctx = np.zeros(B, np.int64)
    q = np.ones(B, np.int64)
    for b in range(n_prefill):
        ctx[b] = rng.bounded(max_prefill_ctx + 1)
        q[b] = chunk
    lens = np.minimum(np.maximum(np.rint(gen.lognormal(np.log(median_len), sigma, n_decode)), 1),
                      max_len).astype(np.int64)
    ctx[n_prefill:] = lens - 1
    k_len = ctx + q
    share_pages = prefix_tokens // page_size
    if n_share is None:
        n_share = B // 2
    sharers = [b for b in range(B) if ctx[b] >= share_pages * page_size][:n_share]
    shared = np.zeros(B, bool)
    shared[sharers] = share_pages > 0
    need = (k_len + page_size - 1) // page_size
    own = need - np.where(shared, share_pages, 0)
    P = int(own.sum()) + (share_pages if shared.any() else 0)
    perm = list(range(P))
    for i in range(P - 1, 0, -1):  # Fisher-Yates with the reference Rng
        j = rng.bounded(i + 1)
        perm[i], perm[j] = perm[j], perm[i]
    pool = iter(perm)
    prefix_ids = [next(pool) for _ in range(share_pages)] if shared.any() else []
    lists = []
    for b in range(B):
        lst = list(prefix_ids) if shared[b] else []
        lst += [next(pool) for _ in range(int(own[b]))]
        lists.append(lst)
    page_ids = np.array([p for lst in lists for p in lst], np.int32)
    cu_pages = np.concatenate([[0], np.cumsum([len(x) for x in lists])]).astype(np.int32)
    rec = page_size * (kv_rank + rope_dim)
    pages = np.empty((n_layers, P, rec), np.uint16)
    for l in range(n_layers):
        pages[l] = to_bits(gen.standard_normal((P, rec), dtype=np.float32), dtype)
    rows = int(q.sum())
    q_latent = to_bits(gen.standard_normal((rows, n_heads, kv_rank), dtype=np.float32), dtype)
    q_rope = to_bits(gen.standard_normal((rows, n_heads, rope_dim), dtype=np.float32), dtype)
    return DecodeBatch(ctx_len=ctx.astype(np.int32), q_len=q.astype(np.int32),
                       cu_pages=cu_pages, page_ids=page_ids, num_pages=P,
                       max_pages=int(need.max()) if B else 0, pages=pages, q_latent=q_latent,
                       q_rope=q_rope, page_size=page_size, kv_rank=kv_rank, rope_dim=rope_dim,
                       n_heads=n_heads, dtype=dtype)


def deepseek_decode_shape(B=256, min_len=8192, max_len=32768, seed=0) -> DecodeBatch:
    """Config 5's batch SHAPE (kernel-only decode at the DeepSeek-like latent shape: 128
    heads, kv_rank 512, rope 64, bf16, 64-token pages): lengths uniform in [8192, 32768]
    and the page permutation from the reference Rng; no contents (6 GB: callers draw
    them on the device)."""
    return ragged_decode_batch(B=B, min_len=min_len, max_len=max_len, n_heads=128,
                               kv_rank=512, rope_dim=64, n_layers=0, dtype=1, seed=seed,
                               q_rows=0)


# mla36m-v1 (config/mla36m-v1.json of the reference), max_sequence_length raised so a
# session can hold config 3's 4096-token contexts (legal up to 65535, config.cpp:21-34).
MLA36M = dict(vocab_size=16384, max_sequence_length=4608, n_layers=10, d_model=512, n_heads=8,
              head_dim_nope=48, head_dim_rope=16, head_dim_value=64, q_lora_rank=192,
              kv_lora_rank=128, d_ff=1360, norm_epsilon=1e-5, rope_theta=10000.0)


def parameter_shapes(cfg: dict):
    """(rows, cols) of every tensor in the reference registry order
    (include/mini_mla/model.hpp:15-30, src/model/model.cpp:40-63)."""
    d, q, kv, H = cfg["d_model"], cfg["q_lora_rank"], cfg["kv_lora_rank"], cfg["n_heads"]
    nope, rope, dv, ff = (cfg["head_dim_nope"], cfg["head_dim_rope"], cfg["head_dim_value"],
                          cfg["d_ff"])
    shapes = [(cfg["vocab_size"], d), (1, d)]
    for _ in range(cfg["n_layers"]):
        shapes += [(1, d), (d, q), (1, q), (q, H * (nope + rope)), (d, kv + rope), (1, kv),
                   (kv, H * nope), (kv, H * dv), (H * dv, d), (1, d), (d, ff), (d, ff), (ff, d)]
    return shapes


def model_params(cfg: dict, seed: int = 0) -> np.ndarray:
    """Random-init parameters with Model::create's scales (src/model/model.cpp:20-75):
    N(0, 0.02), the residual projections w_o and w_down scaled by 1/sqrt(2L), norms 1.
    Drawn from numpy's generator (the reference draws them from its own Rng), in fp32."""
    gen = np.random.default_rng(seed)
    out = []
    resid = 0.02 / np.sqrt(2 * cfg["n_layers"])
    for i, (r, c) in enumerate(parameter_shapes(cfg)):
        slot = -1 if i < 2 else (i - 2) % 13
        if i == 1 or slot in (0, 2, 5, 9):  # final_norm, attn/q/kv/ffn norms
            out.append(np.ones(r * c, np.float32))
        else:
            scale = resid if slot in (8, 12) else 0.02
            out.append((gen.standard_normal(r * c, dtype=np.float32) * scale).astype(np.float32))
    return np.concatenate(out)
