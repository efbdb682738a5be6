"""ctypes binding of the CPU parity oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` -- never by the product package.  The C
restatement cites the reference file:line of each function it follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_RNG = os.path.join(HERE, "_ref", "rng_ref")


class Config(C.Structure):
    """Mirror of ModelConfig's fields (include/mini_mla/model_config.hpp:5-9)."""

    _fields_ = [(n, C.c_int) for n in (
        "vocab_size", "max_sequence_length", "n_layers", "d_model", "n_heads",
        "head_dim_nope", "head_dim_rope", "head_dim_value", "q_lora_rank",
        "kv_lora_rank", "d_ff")] + [("norm_epsilon", C.c_float), ("rope_theta", C.c_float)]

    @classmethod
    def from_dict(cls, d: dict) -> "Config":
        c = cls()
        for name, _ in cls._fields_:
            setattr(c, name, d[name])
        return c

    def to_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}

    @property
    def qk_dim(self) -> int:
        return self.head_dim_nope + self.head_dim_rope


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def _declare(L):
    vp, i, f, u64 = C.c_void_p, C.c_int, C.c_float, C.c_uint64
    sig = {
        "orc_rng_next": (u64, [vp]),
        "orc_rng_uniform": (f, [vp]),
        "orc_rng_bounded": (u64, [vp, u64]),
        "orc_rng_normal": (f, [vp]),
        "orc_rng_fill_normal": (None, [vp, vp, C.c_size_t]),
        "orc_rng_fill_bounded": (None, [vp, u64, vp, C.c_size_t]),
        "orc_f32_to_f16": (C.c_uint16, [f]),
        "orc_round_f16": (None, [vp, vp, C.c_size_t]),
        "orc_round_bf16": (None, [vp, vp, C.c_size_t]),
        "orc_parameter_count": (C.c_size_t, [vp]),
        "orc_validate": (i, [vp]),
        "orc_parameter_shapes": (i, [vp, vp, vp]),
        "orc_model_init": (i, [vp, u64, vp]),
        "orc_forward": (i, [vp, vp, vp, i, vp, vp, vp]),
        "orc_output_projection": (None, [vp, vp, vp]),
        "orc_decode": (i, [vp, vp, vp, vp, vp, i, C.c_uint16, i, i, vp]),
        "orc_set_threads": (None, [i]),
        "orc_set_blas": (None, [vp, vp]),
        "orc_attention_paged": (i, [i, i, i, i, i, i, vp, vp, vp, i, vp, vp, vp, f, vp, vp]),
        "orc_build_metadata": (i, [i, vp, vp, vp, vp, i, i, i, i, i, i, i, i,
                                   vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
        "orc_append_paged": (None, [i, i, i, i, i, vp, vp, vp, vp]),
        "orc_greedy": (i, [vp, i, vp, i, f, vp, i]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


# ---------------------------------------------------------------- Rng ----
class Rng:
    """include/mini_mla/rng.hpp:7-38 through the C restatement."""

    def __init__(self, seed: int = 42):
        self.state = np.array([seed], dtype=np.uint64)

    def next(self) -> int:
        return int(lib().orc_rng_next(_p(self.state)))

    def uniform(self) -> float:
        return float(lib().orc_rng_uniform(_p(self.state)))

    def bounded(self, bound: int) -> int:
        return int(lib().orc_rng_bounded(_p(self.state), bound))

    def normal(self) -> float:
        return float(lib().orc_rng_normal(_p(self.state)))

    def normals(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        lib().orc_rng_fill_normal(_p(self.state), _p(out), n)
        return out

    def bounded_many(self, bound: int, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.int32)
        lib().orc_rng_fill_bounded(_p(self.state), bound, _p(out), n)
        return out


def round_f16(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 bits (uint16), IEEE RNE (src/core/io.cpp:152-158)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_round_f16(_p(x), _p(out), x.size)
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_round_bf16(_p(x), _p(out), x.size)
    return out


def bits_to_f32(bits: np.ndarray, dtype: int = 0) -> np.ndarray:
    if dtype == 0:
        return bits.view(np.float16).astype(np.float32)
    return (bits.astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------- model ----
def parameter_count(cfg: Config) -> int:
    return int(lib().orc_parameter_count(C.byref(cfg)))


def validate(cfg: Config) -> bool:
    return lib().orc_validate(C.byref(cfg)) == 0


def parameter_shapes(cfg: Config):
    n = 2 + 13 * cfg.n_layers
    rows = np.zeros(n, np.int32)
    cols = np.zeros(n, np.int32)
    lib().orc_parameter_shapes(C.byref(cfg), _p(rows), _p(cols))
    return list(zip(rows.tolist(), cols.tolist()))


def model_init(cfg: Config, seed: int) -> np.ndarray:
    params = np.empty(parameter_count(cfg), dtype=np.float32)
    if lib().orc_model_init(C.byref(cfg), seed, _p(params)):
        raise ValueError("invalid config")
    return params


def forward(cfg: Config, params: np.ndarray, tokens, want_cache: bool = False):
    tokens = np.ascontiguousarray(tokens, dtype=np.uint16)
    T = tokens.size
    logits = np.empty((T, cfg.vocab_size), np.float32)
    ckv = np.empty((cfg.n_layers, T, cfg.kv_lora_rank), np.float32) if want_cache else None
    kr = np.empty((cfg.n_layers, T, cfg.head_dim_rope), np.float32) if want_cache else None
    st = lib().orc_forward(C.byref(cfg), _p(params), _p(tokens), T, _p(logits), _p(ckv), _p(kr))
    if st:
        raise ValueError(f"forward failed ({st})")
    return (logits, ckv, kr) if want_cache else logits


def output_projection(cfg: Config, params: np.ndarray) -> np.ndarray:
    out = np.empty((cfg.n_layers, cfg.n_heads * cfg.kv_lora_rank, cfg.d_model), np.float32)
    lib().orc_output_projection(C.byref(cfg), _p(params), _p(out))
    return out


class Decoder:
    """CpuDecoder (src/infer/inference.cpp:10-174) with a contiguous fp32 cache."""

    def __init__(self, cfg: Config, params: np.ndarray, absorbed: bool = True,
                 round_cache: bool = False, proj: np.ndarray | None = None):
        self.cfg, self.params = cfg, params
        self.absorbed, self.round_cache = absorbed, round_cache
        # prepare_projections' result may be shared between decoders of one model
        self.proj = output_projection(cfg, params) if proj is None else proj
        S = cfg.max_sequence_length
        self.latent = np.zeros((cfg.n_layers, S, cfg.kv_lora_rank), np.float32)
        self.rope = np.zeros((cfg.n_layers, S, cfg.head_dim_rope), np.float32)
        self.position = 0

    def prefill(self, ids) -> np.ndarray:
        """CpuDecoder::prefill (inference.cpp:47-68)."""
        self.position = 0
        ids = list(ids)
        if not ids or len(ids) > self.cfg.max_sequence_length:
            raise ValueError("Prompt exceeds context or is empty")
        logits, ckv, kr = forward(self.cfg, self.params, ids, want_cache=True)
        T = len(ids)
        if self.round_cache:
            ckv = bits_to_f32(round_f16(ckv))
            kr = bits_to_f32(round_f16(kr))
        self.latent[:, :T] = ckv
        self.rope[:, :T] = kr
        self.position = T
        return logits[-1].copy()

    def decode(self, token: int) -> np.ndarray:
        logits = np.empty(self.cfg.vocab_size, np.float32)
        st = lib().orc_decode(C.byref(self.cfg), _p(self.params), _p(self.proj),
                              _p(self.latent), _p(self.rope), self.position, token,
                              int(self.absorbed), int(self.round_cache), _p(logits))
        if st:
            raise ValueError(f"decode failed ({st})")
        self.position += 1
        return logits


# -------------------------------------------------------------- CBLAS ----
_blas = None


def use_blas(enable: bool = True):
    """Route orc_forward / orc_decode's products through the CBLAS numpy ships (OpenBLAS,
    64-bit indices) in place of the plain loops -- the portable stand-in for the
    reference's Accelerate cblas calls, used to time the CPU baseline.  The library runs
    single-threaded per call (one session per thread, as the reference's forks decode).
    Returns a description of the library, or None when disabled or not found."""
    global _blas
    import glob
    if not enable:
        lib().orc_set_blas(None, None)
        return None
    if _blas is None:
        libs = sorted(glob.glob(os.path.join(os.path.dirname(np.__file__) + ".libs",
                                             "libscipy_openblas64_*.so")))
        if not libs:
            return None
        B = C.CDLL(libs[0])
        B.scipy_openblas_set_num_threads64_.argtypes = [C.c_int]
        B.scipy_openblas_set_num_threads64_(1)
        B.scipy_openblas_get_config64_.restype = C.c_char_p
        _blas = (B, B.scipy_openblas_get_config64_().decode())
    B, desc = _blas
    lib().orc_set_blas(C.cast(B.scipy_cblas_sgemm64_, C.c_void_p),
                       C.cast(B.scipy_cblas_sgemv64_, C.c_void_p))
    return desc


# --------------------------------------------------- paged attention ----
def attention_paged(H, kv_rank, rope_dim, page_size, dtype, cu_q, k_len, page_table, pages,
                    q_latent, q_rope, scale, want_lse=False, threads=1):
    cu_q = np.ascontiguousarray(cu_q, np.int32)
    k_len = np.ascontiguousarray(k_len, np.int32)
    page_table = np.ascontiguousarray(page_table, np.int32)
    pages = np.ascontiguousarray(pages, np.uint16)
    q_latent = np.ascontiguousarray(q_latent, np.float32)
    q_rope = np.ascontiguousarray(q_rope, np.float32)
    B = k_len.size
    rows = int(cu_q[-1])
    out = np.zeros((rows, H, kv_rank), np.float32)
    lse = np.zeros((rows, H), np.float32) if want_lse else None
    lib().orc_set_threads(int(threads))
    st = lib().orc_attention_paged(B, H, kv_rank, rope_dim, page_size, dtype, _p(cu_q),
                                   _p(k_len), _p(page_table), page_table.shape[1], _p(pages),
                                   _p(q_latent), _p(q_rope), float(scale), _p(out), _p(lse))
    if st:
        raise ValueError("attention_paged: invalid arguments")
    return (out, lse) if want_lse else out


def build_metadata(ctx_len, q_len, cu_pages, page_ids, page_size, max_pages, num_pool_pages,
                   split_pages=0, target_blocks=512, max_work=65535, max_rows=1 << 30,
                   placement_xcds=0):
    """The metadata of mla_build_metadata.  Session order (placement_xcds = 0):
    work_session / work_split are cut to the W items.  XCD placement (n > 0): they keep
    all max_work slots, meaningful where ``occupied`` (work_desc session >= 0)."""
    ctx_len = np.ascontiguousarray(ctx_len, np.int32)
    q_len = np.ascontiguousarray(q_len, np.int32)
    cu_pages = np.ascontiguousarray(cu_pages, np.int32)
    page_ids = np.ascontiguousarray(page_ids, np.int32)
    B = ctx_len.size
    total_q = int(q_len.sum())
    out = dict(
        cu_seqlens_q=np.zeros(B + 1, np.int32), cu_seqlens_k=np.zeros(B + 1, np.int32),
        page_table=np.zeros((B, max_pages), np.int32), slot_mapping=np.zeros(total_q, np.int32),
        num_splits=np.zeros(B, np.int32), cu_splits=np.zeros(B + 1, np.int32),
        work_session=np.zeros(max_work, np.int32), work_split=np.zeros(max_work, np.int32),
        work_desc=np.zeros((max_work, 8), np.int32), work_pages=np.zeros((max_work, 8), np.int32),
        info=np.zeros(8, np.int32))
    st = lib().orc_build_metadata(
        B, _p(ctx_len), _p(q_len), _p(cu_pages), _p(page_ids if page_ids.size else
                                                    np.zeros(1, np.int32)),
        page_size, max_pages, num_pool_pages, split_pages, target_blocks, max_work, max_rows,
        placement_xcds, *(_p(out[k]) for k in ("cu_seqlens_q", "cu_seqlens_k", "page_table", "slot_mapping",
                               "num_splits", "cu_splits", "work_session", "work_split",
                               "work_desc", "work_pages", "info")))
    if st:
        raise ValueError(f"invalid metadata input (session {int(out['info'][1])})")
    W = int(out["info"][0])
    out["occupied"] = out["work_desc"][:, 0] >= 0
    if placement_xcds == 0:
        out["work_session"] = out["work_session"][:W]
        out["work_split"] = out["work_split"][:W]
    return out


def append_paged(kv_rank, rope_dim, page_size, dtype, ckv, krope, slot_mapping, pages):
    ckv = np.ascontiguousarray(ckv, np.float32)
    krope = np.ascontiguousarray(krope, np.float32)
    slot_mapping = np.ascontiguousarray(slot_mapping, np.int32)
    assert pages.flags.c_contiguous and pages.dtype == np.uint16
    lib().orc_append_paged(slot_mapping.size, kv_rank, rope_dim, page_size, dtype, _p(ckv),
                           _p(krope), _p(slot_mapping), _p(pages))


def greedy(logits, history=(), repetition_penalty=1.0, banned=()) -> int:
    logits = np.ascontiguousarray(logits, np.float32)
    h = np.ascontiguousarray(np.array(history, np.uint16).reshape(-1))
    b = np.ascontiguousarray(np.array(banned, np.uint16).reshape(-1))
    return int(lib().orc_greedy(_p(logits), logits.size, _p(h), h.size,
                                float(repetition_penalty), _p(b), b.size))


def ref_rng(kind: str, seed: int, count: int, bound: int = 0):
    """Run the reference's own Rng (oracle/_ref/rng_ref) when it was built."""
    if not os.path.exists(REF_RNG):
        return None
    out = subprocess.run([REF_RNG, kind, str(seed), str(count), str(bound)], check=True,
                         capture_output=True, text=True).stdout.split()
    return out
