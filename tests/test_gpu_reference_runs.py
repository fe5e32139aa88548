"""The reference's own programs on this backend, end to end.

oracle/_ref/ntc_ref_main is the reference's main.cpp built as its CMakeLists.txt builds the CPU trainer;
oracle/_ref/ntc_hip_main is the same main.cpp compiled with NTC_CUDA=1 against include/ntc_cuda.h and
linked against libntc_hip.so (oracle/Makefile, targets programs and drop-in). oracle/_ref/inputs holds the
reference's own test images (make inputs).

* test_cpu_gpu_trajectory: the reference's CPU trainer and its --cuda trainer on this backend, same
  flags, same seed, --rng hash (both draw the same perturbations and minibatches, and the same host
  initialisation), must print the same PSNR at every progress line to 0.05 dB - the reference's own
  cross-backend check (README.md:964-970: 38.24 dB GPU vs 38.23 dB CPU after 300 iterations).
* test_published_run: the command lines of the reference's published GPU runs (README.md:358, 382,
  643, 653, 666), on the images they were published on, run to the end on this backend; the final PSNR
  is within the seed spread of the published one (the host initialisation draws from std::mt19937 and
  std::normal_distribution, whose values differ between the MSVC build the figures come from and this
  one), and the wall time is printed beside the published RTX 5090 time."""
import os
import re
import subprocess

import numpy as np
import pytest

from neural_block_textures_amd import synth
from tests.gpu_common import say
from tests.test_gpu_reference_harness import write_png

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_DIR = os.path.join(ROOT, "oracle", "_ref")
GPU_EXE, CPU_EXE = os.path.join(REF_DIR, "ntc_hip_main"), os.path.join(REF_DIR, "ntc_ref_main")
INPUTS = os.path.join(REF_DIR, "inputs")
PSNR = re.compile(r"^iter\s+(\d+)\s+mse\s+([0-9.]+)\s+psnr\s+([0-9.]+) dB")
DONE = re.compile(r"^done: final psnr ([0-9.]+) dB.*\| ([0-9.]+)s$")


def image(tmp_path, name, size):
    """a crop of the reference's image when it is staged, else a synthetic texture of the same size"""
    src = os.path.join(INPUTS, name)
    dst = str(tmp_path / f"crop_{size}_{name}")
    try:
        from PIL import Image
        rgb = np.asarray(Image.open(src).convert("RGB"))[:size, :size]
    except Exception:
        rgb = synth.rgb_texture(41, size, size)
    write_png(dst, np.ascontiguousarray(rgb))
    return dst


def progress(out):
    return [(int(m.group(1)), float(m.group(2)), float(m.group(3))) for m in map(PSNR.match, out.splitlines()) if m]


TRAJ = {
    # README.md:956-970's check: 3,1-bit selectors + a 4-channel block latent, 36,36 (on a 256x256 crop)
    "qat31": "--latent 256 256 2 --latent2 64 64 4 --filter nearest,nearest --pos lv1local --qat 3,1 --mlp 36,36 --iters 200",
    # README.md:358's flags (annealing, the switch to central differences at half time) on a 256x256 crop
    "qat2_fd": ("--latent 256 256 1 --latent2 64 64 2 --filter nearest,nearest --pos lv1local --qat 2 --mlp 36,36 --mlp-pairs 64 "
                "--iters 200 --lr-anneal 0.5 0.05 --mlp-fd 0.5 --leak 0.0009765625"),
    # a DCT-coded plane with its refit and rate proxy, --qes on the block latent, 17,17 (README.md:653 on a crop)
    "dct_qes": ("--block 8 --latent 0 0 1 --latent2 0 0 4 --filter nearest,bilinear --pos lv1local --dct-q 50 --dct-start 0 "
                "--dct-refit 50 --qes 0,8 --qes-start 0 --mlp 17,17 --mlp-pairs 64 --iters 150 --leak 0.0009765625"),
}


@pytest.mark.skipif(not (os.path.exists(GPU_EXE) and os.path.exists(CPU_EXE)),
                    reason="the reference's programs are built only where the reference tree is present")
@pytest.mark.parametrize("name", list(TRAJ))
def test_cpu_gpu_trajectory(tmp_path, name):
    png = image(tmp_path, "chief1.png", 256)
    runs = {}
    for kind, exe, extra in (("gpu", GPU_EXE, ["--cuda"]), ("cpu", CPU_EXE, [])):
        cmd = [exe, png, *extra, *TRAJ[name].split(), "--rng", "hash", "--seed", "7", "--print-every", "25",
               "--out", str(tmp_path / f"out_{kind}")]
        say("reference", kind, name, " ".join(cmd[2:]))
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, (r.stdout + r.stderr)[-3000:]
        runs[kind] = progress(r.stdout)
    g, c = runs["gpu"], runs["cpu"]
    say("\n".join(f"  iter {a[0]:5d}  gpu mse {a[1]:.3f} psnr {a[2]:.2f}   cpu mse {b[1]:.3f} psnr {b[2]:.2f}" for a, b in zip(g, c)))
    assert [a[0] for a in g] == [b[0] for b in c] and len(g) >= 5
    for a, b in zip(g, c):
        assert abs(a[2] - b[2]) <= 0.05, (a, b)


L = "--lr-anneal 0.5 0.05 --mlp-fd 0.5 --leak 0.0009765625"
PUBLISHED = {
    # name: (README line, images, flags, published seconds on the RTX 5090, published PSNR)
    "chief1_qat2_36": ("README.md:358-373", ["chief1.png"], f"--latent 512 512 1 --latent2 128 128 2 --filter nearest,nearest "
                       f"--pos lv1local --qat 2 --mlp 36,36 --mlp-pairs 64 --iters 8000 {L}", 73.0, 34.57),
    "m1234_qat2_36": ("README.md:382-407", ["m1.png", "m2.png", "m3.png", "m4.png"], f"--latent 512 512 2 --latent2 128 128 4 "
                      f"--filter nearest,nearest --pos lv1local --qat 2 --mlp 36,36 --mlp-pairs 64 --iters 8000 {L}", 107.0, 29.39),
    "frymire_dct80_17": ("README.md:638-644", ["frymire.png"], f"--block 6 --latent 0 0 1 --latent2 0 0 4 --filter nearest,bilinear "
                         f"--pos lv1local --dct-q 80 --dct-refit 500 --qes 0,8 --mlp 17,17 --mlp-pairs 256 --iters 8000 {L} "
                         f"--dct-map all --lat-init-image --write-ntcb", 29.1, 32.99),
    "chief1_dct50_17": ("README.md:646-654", ["chief1.png"], f"--block 6 --latent 0 0 1 --latent2 0 0 4 --filter nearest,bilinear "
                        f"--pos lv1local --dct-q 50 --dct-refit 500 --qes 0,8 --mlp 17,17 --mlp-pairs 256 --iters 8000 {L} "
                        f"--dct-map all --lat-init-image --write-ntcb", 15.1, 34.71),
    "chief1_qat3_17": ("README.md:657-667", ["chief1.png"], f"--block 6 --latent 0 0 1 --latent2 0 0 4 --filter nearest,bilinear "
                       f"--pos lv1local --qat 3 --qes 0,8 --mlp 17,17 --mlp-pairs 256 --iters 8000 {L} --lat-init-image --write-ntcb",
                       15.3, 38.53),
}


@pytest.mark.skipif(not (os.path.exists(GPU_EXE) and os.path.isdir(INPUTS)),
                    reason="the reference's program and images are staged only where the reference tree is present")
@pytest.mark.parametrize("name", list(PUBLISHED))
def test_published_run(tmp_path, name):
    src, imgs, flags, pub_s, pub_psnr = PUBLISHED[name]
    cmd = [GPU_EXE, *[os.path.join(INPUTS, i) for i in imgs], "--cuda", *flags.split(), "--out", str(tmp_path / "out")]
    say("published run", name, src, " ".join(cmd[1:]))
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, (r.stdout + r.stderr)[-3000:]
    done = [m for m in map(DONE.match, r.stdout.splitlines()) if m]
    assert done, r.stdout[-3000:]
    psnr, secs = float(done[-1].group(1)), float(done[-1].group(2))
    say(f"published run {name}: {secs:.1f} s on this backend vs {pub_s:.1f} s published (RTX 5090), {pub_s / secs:.1f}x; "
        f"final psnr {psnr:.2f} dB vs {pub_psnr:.2f} dB published")
    assert abs(psnr - pub_psnr) < 1.5
