"""Containers written by the reference itself: its CPU program (oracle/_ref/ntc_ref_main, main.cpp built
by oracle/Makefile target `programs`) trains three small synthetic models with --write-ntcb, and its
standalone decoder (oracle/_ref/ntc_decode, ntc_decode.cpp) decodes each container with --exact. For
every case this keeps

    ntcb_<case>.ntcb         the container (model.ntcb)
    ntcb_<case>_model.bin    the model file the same run saved at its last iteration (the state the
                             container was written from: weights already rounded to fp16)
    ntcb_<case>_images.npz   recon_q_final (the trainer's decode of the container's values) and
                             ntc_decode (the standalone decoder's output of the container), uint8
                             [T][src_h][src_w][3] each

Cases: qat4 (4-texture material, --qat 2 level 0 = palette mode, bilinear level 1 = post-hoc 8-bit
grid), dct (--dct-q 50 level 0 = DCT tokens), qes (--qes 6 on both levels = stored grids, --clamp,
--block padding so the source is smaller than the decode). Run from the repository root where the
reference tree is present, after `make -C oracle programs`:

    python tests/golden/make_ntcb_fixture.py
"""
import os
import shutil
import subprocess
import sys
import tempfile

import numpy as np
from PIL import Image

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from neural_block_textures_amd import synth              # noqa: E402
from neural_block_textures_amd.decode import write_png   # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
MAIN = os.path.join(ROOT, "oracle", "_ref", "ntc_ref_main")
DECODE = os.path.join(ROOT, "oracle", "_ref", "ntc_decode")
COMMON = ["--mlp", "16,16", "--iters", "40", "--seed", "3", "--rng", "hash", "--threads", "4", "--write-ntcb"]
CASES = {
    "qat4": (("material", 64, 64), ["--latent", "64", "64", "2", "--latent2", "16", "16", "4", "--filter", "nearest,bilinear",
                                    "--qat", "2"]),
    "dct": (("rgb", 64, 64), ["--latent", "64", "64", "1", "--latent2", "16", "16", "4", "--filter", "nearest,bilinear",
                              "--dct-q", "50", "--dct-start", "0"]),
    "qes": (("rgb", 60, 44), ["--block", "8", "--latent", "32", "24", "4", "--latent2", "16", "12", "2", "--qes", "6",
                              "--qes-start", "0", "--clamp"]),
}


def images(kind, W, H, d):
    maps = synth.material(21, W, H) if kind == "material" else [synth.rgb_texture(22, W, H)]
    names = []
    for t, m in enumerate(maps):
        names.append(os.path.join(d, f"in{t}.png"))
        write_png(names[-1], m)
    return names


def main():
    for exe in (MAIN, DECODE):
        if not os.path.exists(exe):
            raise SystemExit(f"{exe} is missing: make -C oracle programs")
    for case, ((kind, W, H), flags) in CASES.items():
        with tempfile.TemporaryDirectory() as d:
            ins = images(kind, W, H, d)
            out = os.path.join(d, "out")
            log = subprocess.run([MAIN, *flags, *COMMON, "--out", out, *ins], capture_output=True, text=True, check=True).stdout
            print(case, [ln for ln in log.splitlines() if ln.startswith("file:")][0][:100])
            shutil.copyfile(os.path.join(out, "model.ntcb"), os.path.join(OUT, f"ntcb_{case}.ntcb"))
            shutil.copyfile(os.path.join(out, "model.bin"), os.path.join(OUT, f"ntcb_{case}_model.bin"))
            T = len(ins)
            subprocess.run([DECODE, os.path.join(out, "model.ntcb"), "-o", os.path.join(d, "dec"), "--exact", "--threads", "4"],
                           capture_output=True, text=True, check=True)
            dec = [os.path.join(d, "dec.png")] if T == 1 else [os.path.join(d, f"dec_t{t}.png") for t in range(T)]
            rq = [os.path.join(out, "recon_q_final.png")] if T == 1 else [os.path.join(out, f"recon_q_final_t{t}.png") for t in range(T)]
            load = lambda names: np.stack([np.asarray(Image.open(n).convert("RGB")) for n in names])   # noqa: E731
            np.savez_compressed(os.path.join(OUT, f"ntcb_{case}_images.npz"), recon_q_final=load(rq), ntc_decode=load(dec))
    print("fixtures written to", OUT)


if __name__ == "__main__":
    main()
