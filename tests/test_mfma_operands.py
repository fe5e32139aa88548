"""The library's matrix-core device code as built: no v_mfma_f32_4x4x1_16b_f32 may write registers that partially
overlap its C operand.

The register allocator may give a matrix instruction a destination range that shares some registers with the
accumulator it reads (v[60:63] from v[62:65]). For v_mfma_f32_16x16x4_f32 the kernels are full of such
allocations and every parity test passes with them. For the 4x4x1 instruction on gfx950 one such allocation
made a population kernel's central-difference member losses 21% wrong while the same build's other instances
stayed correct. The kernels keep the 4x4x1 accumulator chains that the allocator has left whole; this test
compiles kernels_pop.hip with the build's own flags and fails if a later change to the sources leads the
compiler to split one."""
import os
import re
import subprocess

import pytest

from neural_block_textures_amd import build as B

MFMA = re.compile(r"^\s*(v_mfma_f32_4x4x1\S*)\s+v\[(\d+):(\d+)\],\s*\S+,\s*\S+,\s*v\[(\d+):(\d+)\]")


def partial_overlaps(asm: str):
    """(kernel, instruction) for every 4x4x1 instruction whose destination and C ranges overlap without being equal"""
    bad, kernel = [], None
    for line in asm.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            kernel = m.group(1)
            continue
        m = MFMA.match(line)
        if not m:
            continue
        d0, d1, c0, c1 = (int(m.group(i)) for i in (2, 3, 4, 5))
        if (d0, d1) != (c0, c1) and not (d1 < c0 or c1 < d0):
            bad.append((kernel, line.strip()))
    return bad


def test_the_checker_finds_a_split_chain():
    asm = ("_Zk:\n\tv_mfma_f32_4x4x1_16b_f32 v[60:63], v33, v60, v[62:65]\n"
           "\tv_mfma_f32_4x4x1_16b_f32 v[14:17], v32, v72, v[14:17]\n"
           "\tv_mfma_f32_4x4x1_16b_f32 v[18:21], v33, v81, 0\n"
           "\tv_mfma_f32_4x4x1_16b_f32 v[22:25], v33, v81, v[26:29]\n")
    assert partial_overlaps(asm) == [("_Zk", "v_mfma_f32_4x4x1_16b_f32 v[60:63], v33, v60, v[62:65]")]


def test_no_4x4x1_with_a_partially_overlapping_accumulator(tmp_path):
    try:
        hipcc = B.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    out = tmp_path / "kernels_pop.s"
    cmd = [hipcc, *B.flags("kernels_pop.hip"), "--offload-device-only", "-S", "-o", str(out),
           os.path.join(B.CSRC, "kernels_pop.hip")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    asm = out.read_text()
    assert "v_mfma_f32_4x4x1" in asm   # the pixel-per-lane output layer is in the library
    bad = partial_overlaps(asm)
    assert not bad, f"{len(bad)} split 4x4x1 accumulator chain(s), e.g. {bad[0]}"
