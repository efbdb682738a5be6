"""Guards on the gfx950 machine code this repository builds (CPU only).

MFMA instructions must not have a destination that partially overlaps their
accumulator input (identical or disjoint only): such a register assignment
corrupted the decode kernel's scores.
"""
import glob
import os
import re
import subprocess

import pytest

from conftest import REPO

CSRC = os.path.join(REPO, "cpp_inference_train_engine_amd", "csrc")


def _asm(src, tmp_path):
    out = tmp_path / (os.path.basename(src) + ".s")
    cmd = ["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "-std=c++20", "-S",
           "--cuda-device-only", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", os.path.join(REPO, "include"), "-I", CSRC, src, "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        pytest.fail(res.stderr[-2000:])
    return out.read_text()


def _reg_range(tok):
    m = re.match(r"([av])\[(\d+):(\d+)\]", tok)
    if m:
        return m.group(1), int(m.group(2)), int(m.group(3))
    m = re.match(r"([av])(\d+)$", tok)
    if m:
        return m.group(1), int(m.group(2)), int(m.group(2))
    return None


def mfma_partial_overlaps(asm: str):
    bad = []
    for line in asm.splitlines():
        if "v_mfma" not in line:
            continue
        ops = [o.strip() for o in line.split(None, 1)[1].split(",")]
        if len(ops) < 4:
            continue
        d, c = _reg_range(ops[0]), _reg_range(ops[3])
        if d and c and d[0] == c[0] and (d[1], d[2]) != (c[1], c[2]) and \
                not (d[2] < c[1] or c[2] < d[1]):
            bad.append(line.strip())
    return bad


def test_overlap_checker_flags_the_bad_form():
    asm = "\tv_mfma_f32_16x16x16_f16 a[2:5], v[56:57], v[134:135], a[4:7]\n" \
          "\tv_mfma_f32_16x16x32_f16 a[4:7], v[2:5], v[6:9], a[4:7]\n" \
          "\tv_mfma_f32_16x16x32_f16 a[0:3], v[2:5], v[6:9], 0\n"
    assert len(mfma_partial_overlaps(asm)) == 1


@pytest.mark.parametrize("src", sorted(glob.glob(os.path.join(CSRC, "*.hip"))),
                         ids=os.path.basename)
def test_no_mfma_partial_dst_src_overlap(src, tmp_path):
    assert mfma_partial_overlaps(_asm(src, tmp_path)) == []
