"""The reference's own GPU-vs-CPU harness against this backend.

oracle/_ref/ntc_hip_main is the reference's main.cpp, compiled unmodified with NTC_CUDA=1 against
include/ntc_cuda.h and linked against libntc_hip.so (oracle/Makefile, target drop-in). With
`--cuda --cuda-check` it runs its seven comparisons (main.cpp:2983-3219) - decode, MLP ES pair
differences, central differences, the latent gradient (and the --dct-lambda integers), the qat
search, the --qes snapped copy, and the DCT symbols / plane / codes with a refit - against its own
CPU code on identical inputs, and prints PASS or FAIL per item. The inputs are synthetic PNGs."""
import os
import struct
import subprocess
import zlib

import numpy as np
import pytest

from neural_block_textures_amd import synth
from tests.gpu_common import say

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "oracle", "_ref", "ntc_hip_main")


def write_png(path, rgb):
    """8-bit RGB PNG (filter 0 on every row)."""
    h, w, _ = rgb.shape
    raw = b"".join(b"\x00" + rgb[y].tobytes() for y in range(h))

    def chunk(tag, data):
        return struct.pack(">I", len(data)) + tag + data + struct.pack(">I", zlib.crc32(tag + data) & 0xFFFFFFFF)

    png = b"\x89PNG\r\n\x1a\n" + chunk(b"IHDR", struct.pack(">IIBBBBB", w, h, 8, 2, 0, 0, 0))
    png += chunk(b"IDAT", zlib.compress(raw, 6)) + chunk(b"IEND", b"")
    with open(path, "wb") as f:
        f.write(png)


CASES = {
    "default": (1, "--latent 16 16 4 --mlp 16,16"),
    "two_level": (1, "--latent 32 32 8 --latent2 8 8 4 --mlp 32,32 --leak 0"),
    "lv1local_clamp": (1, "--latent 16 16 4 --latent2 6 6 2 --pos uv,lv1local --mlp 20,12 --clamp"),
    "material_qat": (4, "--latent 64 64 2 --latent2 16 16 4 --filter nearest,bilinear --qat 2 --mlp 32,32 --weights 1,2,1,1"),
    "qes": (1, "--latent 32 32 4 --latent2 8 8 4 --qes 5 --qes-start 0 --mlp 24,24"),
    "dct": (1, "--latent 64 64 1 --latent2 16 16 4 --filter nearest,bilinear --dct-q 50 --dct-start 0 --dct-lambda 0 --mlp 32,32"),
    "dct_lambda": (1, "--latent 64 64 2 --latent2 16 16 4 --filter nearest,bilinear --dct-q 75,40 --dct-start 0 --dct-lambda 0.5 --mlp 24,24"),
    "dct_deadzone_trunc": (1, "--latent 64 64 1 --latent2 16 16 4 --filter nearest,bilinear --dct-q 30 --dct-start 0 --dct-deadzone 1 --dct-lambda 0.4 --dct-rate trunc --mlp 16,16"),
}


@pytest.mark.skipif(not os.path.exists(EXE), reason="oracle/_ref/ntc_hip_main is built only where the reference tree is present")
@pytest.mark.parametrize("name", list(CASES))
def test_reference_cuda_check(tmp_path, name):
    ntex, flags = CASES[name]
    pngs = []
    if ntex == 4:
        maps = synth.material(31, 64, 64)
    else:
        maps = [synth.rgb_texture(31, 64, 64)]
    for t, m in enumerate(maps):
        pth = str(tmp_path / f"t{t}.png")
        write_png(pth, np.ascontiguousarray(m))
        pngs.append(pth)
    cmd = [EXE, *pngs, "--cuda", "--cuda-check", "--rng", "hash", "--out", str(tmp_path / "out"), "--mlp-batch", "2048",
           "--seed", "3", *flags.split()]
    say("reference harness:", name, " ".join(cmd[1:]))
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=240)
    out = r.stdout + r.stderr
    lines = [l for l in out.splitlines() if l.strip().startswith(("decode", "mlp", "latent", "qat", "qes", "dct", "cuda-check"))]
    say("\n".join(lines))
    assert r.returncode == 0, out[-3000:]
    assert "cuda-check: all passed" in out
    assert "FAIL" not in out


# The reference's own check lines (README.md:1117-1126), verbatim, on its own images (oracle/_ref/inputs,
# staged by `make -C oracle inputs`), plus the variants its comments name (--dct-q 90 and 20,
# --dct-lambda 100000, the two-channel --dct-lambda line with --dct-deadzone 0).
INPUTS = os.path.join(ROOT, "oracle", "_ref", "inputs")
_BLK8 = "--block 8 --latent 0 0 1 --latent2 0 0 4 --filter nearest,bilinear --pos lv1local"
_BLK4 = "--block 4 --latent 0 0 2 --latent2 0 0 4 --filter nearest,bilinear --pos lv1local"
_DCT = "--dct-shadow-pull 0 --dct-start 0 --qes 0,8 --qes-start 0"
_TAIL = "--leak 0.0009765625 --iters 5 --print-every 5"
README_CHECKS = {
    "1117_qat31": "chief1.png --latent 512 512 2 --latent2 128 128 4 --filter nearest,nearest --pos lv1local --qat 3,1 --mlp 36,36 --iters 1",
    "1118_default": "--iters 1",
    "1119_m1234_qat2": "m1.png m2.png m3.png m4.png --latent 512 512 3 --latent2 128 128 4 --filter nearest,nearest --pos lv1local --qat 2 --mlp 36,36 --iters 1",
    "1120_qes_block": f"chief1.png {_BLK8} --qat 2 --qes 0,8 --qes-start 0 --mlp 17,17 {_TAIL}",
    "1121_qes_levels": "chief1.png --latent 128 128 4 --latent2 32 32 4 --filter bilinear,bilinear --pos uv --qes 6,8 --qes-start 0 --mlp 17,17 --iters 5 --print-every 5",
    "1122_dct50": f"chief1.png {_BLK8} --dct-deadzone 1 {_DCT} --dct-q 50 --dct-lambda 0 --mlp 17,17 {_TAIL}",
    "1122_dct90": f"chief1.png {_BLK8} --dct-deadzone 1 {_DCT} --dct-q 90 --dct-lambda 0 --mlp 17,17 {_TAIL}",
    "1122_dct20": f"chief1.png {_BLK8} --dct-deadzone 1 {_DCT} --dct-q 20 --dct-lambda 0 --mlp 17,17 {_TAIL}",
    "1123_dct2ch": f"m1.png {_BLK4} --dct-deadzone 1 {_DCT} --dct-q 50,20 --dct-lambda 0 --mlp 27,27 {_TAIL}",
    "1124_dct_lambda": f"chief1.png {_BLK8} --dct-deadzone 1 {_DCT} --dct-q 50 --mlp 17,17 {_TAIL} --dct-lambda 80",
    "1124_dct_lambda_dc_only": f"chief1.png {_BLK8} --dct-deadzone 1 {_DCT} --dct-q 50 --mlp 17,17 {_TAIL} --dct-lambda 100000",
    "1125_dct2ch_lambda": f"m1.png {_BLK4} --dct-deadzone 1 {_DCT} --dct-q 50,20 --mlp 27,27 {_TAIL} --dct-lambda 80",
    "1126_dct_dz0": f"chief1.png {_BLK8} {_DCT} --dct-q 50 --dct-lambda 0 --mlp 17,17 {_TAIL} --dct-deadzone 0",
    "1126_dct2ch_lambda_dz0": f"m1.png {_BLK4} {_DCT} --dct-q 50,20 --mlp 27,27 {_TAIL} --dct-lambda 80 --dct-deadzone 0",
}


@pytest.mark.skipif(not (os.path.exists(EXE) and os.path.isdir(INPUTS)),
                    reason="the reference's program and images are staged only where the reference tree is present")
@pytest.mark.parametrize("name", list(README_CHECKS))
def test_reference_readme_check(tmp_path, name):
    args = README_CHECKS[name].split()
    cmd = [EXE, *args, "--cuda", "--cuda-check", "--out", str(tmp_path / "out_chk")]
    say("reference README check:", name, " ".join(cmd[1:]))
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300, cwd=INPUTS)
    out = r.stdout + r.stderr
    lines = [l for l in out.splitlines() if l.strip().startswith(("decode", "mlp", "latent", "qat", "qes", "dct", "cuda-check"))]
    say("\n".join(lines))
    assert r.returncode == 0, out[-3000:]
    assert "cuda-check: all passed" in out
    assert "FAIL" not in out
