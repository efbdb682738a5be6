"""mla_decode_attention_noalloc: the decode attention call that allocates nothing (its
split partials live in the library's per-GPU scratch array), checked against
mla_decode_attention with a caller workspace on the same inputs -- the same kernels, so
the outputs must be bit-identical.  Two calls in a row, the second with a smaller batch
(the scratch keeps the first call's partials; nothing of them may leak into the second),
the same two over XCD-placed metadata with the merge inside the decode launch (its
counters live in the scratch as well), then a size beyond the scratch maximum, rejected on
the host before any launch."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _entry(lib):
    f = lib.mla_decode_attention_noalloc
    f.restype = C.c_int
    f.argtypes = ([C.c_void_p] + [C.c_int] * 6 + [C.c_float] + [C.c_void_p] * 2 +
                  [C.c_int] * 2 + [C.c_void_p] * 8 + [C.c_int, C.c_void_p, C.c_void_p, C.c_int])
    return f


def _call(gpu, f, B, seed, max_len, placed=False):
    import torch
    from cpp_inference_train_engine_amd.workloads import ragged_decode_batch
    batch = ragged_decode_batch(B=B, min_len=1, max_len=max_len, seed=seed)
    _say(f"noalloc call: B={B} seed={seed} tokens={int(batch.k_len.sum())} placed={placed}")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    rb = gpu.build_metadata(dev(batch.ctx_len), dev(batch.q_len), dev(batch.cu_pages),
                            dev(batch.page_ids), 64, batch.max_pages, batch.num_pages,
                            split_pages=4, placement=placed)
    pages = dev(batch.pages[0].view(np.int16)).view(torch.float16)
    ql = dev(batch.q_latent.view(np.int16)).view(torch.float16)
    qr = dev(batch.q_rope.view(np.int16)).view(torch.float16)
    lse_ref = torch.zeros((B, 8), dtype=torch.float32, device="cuda")
    ref = gpu.decode_attention(rb, pages, ql, qr, 0.125, kv_rank=128, rope_dim=16, lse=lse_ref)
    out = torch.full((B, 8, 128), float("nan"), dtype=torch.float32, device="cuda")
    lse = torch.full((B, 8), float("nan"), dtype=torch.float32, device="cuda")
    p = gpu.ptr
    gpu.check(f(gpu.stream_handle(), B, 8, 128, 16, 64, gpu.DTYPE_F16, 0.125,
                p(rb.cu_seqlens_q), p(rb.page_table), rb.max_pages, rb.num_pool_pages,
                p(pages), p(ql), p(qr), p(rb.num_splits), p(rb.cu_splits), p(rb.work_desc),
                p(rb.work_pages), p(rb.info), rb.max_work, p(out), p(lse),
                gpu.DECODE_FUSED_MERGE if placed else 0))
    torch.cuda.synchronize()
    info = rb.read_info()
    assert info[0] > B, "the case must have split sessions, whose partials use the scratch"
    assert torch.equal(out, ref), f"B={B}: output differs from mla_decode_attention"
    assert torch.equal(lse, lse_ref), f"B={B}: lse differs from mla_decode_attention"


def test_noalloc_decode_equals_workspace_decode(gpu):
    f = _entry(gpu.lib())
    assert gpu.lib().mla_noalloc_scratch_bytes() == 16 << 20
    _call(gpu, f, 64, 0, 4096)  # config 3's size: 570 work items
    _call(gpu, f, 9, 1, 1500)   # then a smaller batch on the same scratch
    # the one-launch decode over XCD-placed metadata (merge counters in the scratch too)
    _call(gpu, f, 64, 2, 4096, placed=True)
    _call(gpu, f, 9, 3, 1500, placed=True)
    # partials beyond the scratch: rejected on the host, nothing launched
    st = f(None, 64, 128, 512, 64, 64, gpu.DTYPE_BF16, 0.1, None, None, 1, 1,
           *([None] * 8), 6000, None, None, 0)
    assert st == 1 and b"scratch maximum" in gpu.lib().mla_last_error()
