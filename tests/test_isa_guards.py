"""Guards on the gfx950 machine code this repository builds (CPU only).

The legacy 16x16x16 f16/bf16 MFMA forms are kept out of every kernel: a decode
kernel that used v_mfma_f32_16x16x16_f16 with AGPR accumulators (result read back
a few instructions later, destination overlapping the accumulator input) produced
wrong scores on gfx950, while the same math on v_mfma_f32_16x16x32_* is exact.
An isolated hardware probe showed the overlap itself computes correctly, so the
guard pins the instruction form, which is what the kernels avoid.
"""
import glob
import os
import re
import subprocess

import pytest

from conftest import REPO

CSRC = os.path.join(REPO, "cpp_inference_train_engine_amd", "csrc")
LEGACY = re.compile(r"v_mfma_f32_16x16x16_?(f16|bf16)")


def _asm(src, tmp_path):
    out = tmp_path / (os.path.basename(src) + ".s")
    cmd = ["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "-std=c++20", "-S",
           "--cuda-device-only", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", os.path.join(REPO, "include"), "-I", CSRC, src, "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        pytest.fail(res.stderr[-2000:])
    return out.read_text()


def test_guard_pattern_matches_the_legacy_forms():
    assert LEGACY.search("\tv_mfma_f32_16x16x16_f16 a[2:5], v[56:57], v[134:135], a[4:7]")
    assert LEGACY.search("\tv_mfma_f32_16x16x16_bf16 v[2:5], v[6:7], v[6:7], v[2:5]")
    assert not LEGACY.search("\tv_mfma_f32_16x16x32_f16 v[4:7], v[2:5], v[6:9], v[4:7]")


@pytest.mark.parametrize("src", sorted(glob.glob(os.path.join(CSRC, "*.hip"))),
                         ids=os.path.basename)
def test_no_legacy_16x16x16_mfma(src, tmp_path):
    asm = _asm(src, tmp_path)
    bad = [line.strip() for line in asm.splitlines() if LEGACY.search(line)]
    assert bad == []
