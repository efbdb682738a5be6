"""The C-ABI library loads (no GPU needed) and exports every function that
include/*.h declares; host-side argument validation returns the reference's
ErrorCode values without touching the device."""
import ctypes
import glob
import os
import re

import pytest

from conftest import REPO


def declared_functions():
    names = []
    for h in glob.glob(os.path.join(REPO, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(mla_\w+)\s*\(", text, re.M)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("mla_build_metadata", "mla_append_latent", "mla_decode_attention",
                 "mla_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import cpp_inference_train_engine_amd as mla
    lib = ctypes.CDLL(mla.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(mla.exported_symbols()) <= set(declared_functions())


def test_invalid_arguments_are_rejected_on_the_host():
    import cpp_inference_train_engine_amd as mla
    L = mla.lib()
    assert L.mla_abi_version() == 2
    st = L.mla_build_metadata(None, -1, *([None] * 4), 64, 4, 10, 0, 16, 8, 8, 0, *([None] * 11))
    assert st == 1 and b"invalid" in L.mla_last_error()
    st = L.mla_build_metadata(None, 4, *([None] * 4), 64, 4, 10, 0, 16, 70000, 8, 0,
                              *([None] * 11))
    assert st == 1  # max_work above MLA_MAX_WORK
    st = L.mla_build_metadata(None, 4, *([None] * 4), 64, 4, 10, 0, 16, 8, 8, 2, *([None] * 11))
    assert st == 1  # placement is 0 or 1
    st = L.mla_build_metadata(None, 257, *([None] * 4), 64, 4, 10, 0, 16, 8, 8, 1,
                              *([None] * 11))
    assert st == 3 and b"256 sessions" in L.mla_last_error()  # unsupported: B > 256
    for n in (0, 9):  # the explicit placement takes 1..8 XCDs
        st = L.mla_build_metadata_placed(None, 4, *([None] * 4), 64, 4, 10, 0, 16, 8, 8, n,
                                         *([None] * 11))
        assert st == 1 and b"n_xcds" in L.mla_last_error()
    st = L.mla_build_metadata_placed(None, 257, *([None] * 4), 64, 4, 10, 0, 16, 8, 8, 2,
                                     *([None] * 11))
    assert st == 3 and b"256 sessions" in L.mla_last_error()
    st = L.mla_append_latent(None, 4, 128, 16, 64, 7, None, None, None, 10, None)
    assert st == 1
    st = L.mla_decode_attention(None, 4, 8, 128, 16, 64, 0, 0.125, *([None] * 2), 4, 10,
                                *([None] * 8), 16, None, None, None, 0, 0)
    assert st == 1  # null buffers
    # The fused flag needs placed metadata, which holds at most 256 sessions: refused on the
    # host before anything reaches the device (the buffers here are host dummies).
    buf = ctypes.create_string_buffer(1 << 16)
    a = ctypes.addressof(buf)
    a -= a % 256
    a += 256
    st = L.mla_decode_attention(None, 300, 8, 128, 16, 64, 0, 0.125, a, a, 4, 10,
                                *([a] * 8), 16, a, None, a, 1 << 40, mla.DECODE_FUSED_MERGE)
    assert st == 1 and b"MLA_DECODE_FUSED_MERGE" in L.mla_last_error()
    st = L.mla_decode_partials(None, 300, 8, 128, 16, 64, 0, 0.125, a, a, 4, 10,
                               *([a] * 8), 16, a, None, a, 1 << 40, mla.DECODE_FUSED_MERGE)
    assert st == 1 and b"MLA_DECODE_FUSED_MERGE" in L.mla_last_error()
    st = L.mla_decode_status(None, None, 4096, 0, a)
    assert st == 1
    st = L.mla_decode_status(None, a, 1000, 0, a)  # smaller than the workspace head
    assert st == 1
    # The head block (256 int32 counters of the fused merge, the status word at byte 1024,
    # 1280 bytes), then per slot o [H][kv_rank] fp32 and the (m, l) pairs [H][2] padded to
    # 128 bytes, rounded up to 256 bytes; the size does not depend on the session count
    assert mla.DECODE_WORKSPACE_HEAD == 1280 and mla.DECODE_STATUS_OFFSET == 1024
    assert L.mla_decode_workspace_bytes(16, 4, 8, 128) == 1280 + 16 * (8 * 128 + 32) * 4
    assert L.mla_decode_workspace_bytes(3, 4, 17, 128) == 1280 + (3 * (17 * 128 + 64) * 4 + 255) // 256 * 256
    assert L.mla_decode_workspace_bytes(16, 100, 8, 128) == L.mla_decode_workspace_bytes(16, 4, 8,
                                                                                          128)
    with pytest.raises(mla.MlaError) as e:
        mla.check(1)
    assert e.value.code == "invalid_argument"


def test_fused_python_guard_refuses_unplaced_metadata():
    """The operator wrapper refuses fused=True over metadata that is not placed for this
    device before anything reaches the library (CPU: no device call is made)."""
    import torch
    import cpp_inference_train_engine_amd as mla
    rb = mla.RaggedBatch(B=2, page_size=64, max_pages=1, num_pool_pages=2, max_work=2,
                         max_rows=2, **{k: None for k in (
                             "cu_seqlens_q", "cu_seqlens_k", "page_table", "slot_mapping",
                             "num_splits", "cu_splits", "work_session", "work_split",
                             "work_desc", "work_pages", "info")})
    q = torch.zeros((2, 8, 128), dtype=torch.float16)
    with pytest.raises(ValueError, match="placed"):
        mla.decode_attention(rb, None, q, q[:, :, :16], 0.125, kv_rank=128, rope_dim=16,
                             fused=True, workspace=torch.zeros(4, dtype=torch.uint8))
