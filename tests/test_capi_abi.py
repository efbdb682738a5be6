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
    assert L.mla_abi_version() == 1
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
    st = L.mla_append_latent(None, 4, 128, 16, 64, 7, None, None, None, 10, None)
    assert st == 1
    st = L.mla_decode_attention(None, 4, 8, 128, 16, 64, 0, 0.125, *([None] * 2), 4, 10,
                                *([None] * 8), 16, None, None, None, 0, 0)
    assert st == 1  # null buffers
    # 256 int32 counters of the fused merge, then per slot o [H][kv_rank] fp32 and the
    # (m, l) pairs [H][2] padded to 128 bytes, rounded up to 256 bytes; the size does not
    # depend on the session count
    assert L.mla_decode_workspace_bytes(16, 4, 8, 128) == 1024 + 16 * (8 * 128 + 32) * 4
    assert L.mla_decode_workspace_bytes(3, 4, 17, 128) == 1024 + (3 * (17 * 128 + 64) * 4 + 255) // 256 * 256
    assert L.mla_decode_workspace_bytes(16, 100, 8, 128) == L.mla_decode_workspace_bytes(16, 4, 8,
                                                                                          128)
    with pytest.raises(mla.MlaError) as e:
        mla.check(1)
    assert e.value.code == "invalid_argument"
