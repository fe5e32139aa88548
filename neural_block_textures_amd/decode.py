"""Decode a model file of the reference (model.bin v11 .. v14, or the bit-packed model.ntcb) on the GPU
to 8-bit PNGs, one per texture, cropped to the source extent the file records (as ntc_decode writes).

    python -m neural_block_textures_amd.decode model.bin|model.ntcb out_prefix [--repeat 50]

The decode is the trainer's: the latent levels (a DCT-coded level 0 reconstructed from its symbols on
the device), the MLP, and save_png's rounding, all on the device; W x H x 3T bytes cross PCIe. A
container's grid and palette levels are dequantized on the host as its readers do (strict float32).
With --repeat the decode is timed (HIP events around the decode and pack kernels) and reported in
Mtexel/s, the unit of the reference's ntc_decode timings.
"""
from __future__ import annotations

import argparse
import json
import struct
import sys
import time
import zlib

import numpy as np

from . import dct_host, model_file, ntcb
from .trainer import DctDesc, Trainer


def write_png(path: str, rgb: np.ndarray) -> None:
    """8-bit RGB PNG, filter 0 on every row"""
    h, w, _ = rgb.shape
    raw = b"".join(b"\x00" + np.ascontiguousarray(rgb[y]).tobytes() for y in range(h))

    def chunk(tag, data):
        return struct.pack(">I", len(data)) + tag + data + struct.pack(">I", zlib.crc32(tag + data) & 0xFFFFFFFF)

    png = b"\x89PNG\r\n\x1a\n" + chunk(b"IHDR", struct.pack(">IIBBBBB", w, h, 8, 2, 0, 0, 0))
    png += chunk(b"IDAT", zlib.compress(raw, 6)) + chunk(b"IEND", b"")
    with open(path, "wb") as f:
        f.write(png)


def trainer_for(m: model_file.ModelFile) -> Trainer:
    """a trainer holding the file's model (decode only: the target is zero)"""
    lay = m.layout
    if lay.W < 1 or lay.H < 1:
        raise ValueError("the model file carries no image size (v9 / v10): decode needs a v11+ file")
    kw = {}
    if m.dct:
        C0 = lay.levels[0][2]
        kw = dict(dct={"C": C0, "q": m.dct["q"], "dc_step": m.dct["dc_step"]}, dct_basis=dct_host.basis(),
                  dct_zigzag=dct_host.zigzag())
    tr = Trainer()
    tr.init(Trainer.model_desc(lay, max_pairs=1, max_batch=16, **kw), m.z, m.p, np.zeros(lay.W * lay.H * lay.nout, np.float32),
            lay)
    if m.dct:
        W0, H0, C0, _ = lay.levels[0]
        d = DctDesc()
        d.live, d.C, d.BW, d.BH, d.N, d.dc_step = 1, C0, W0 // 8, H0 // 8, 8, m.dct["dc_step"]
        d.lo_w16, d.deadzone = 16, m.dct["deadzone"]
        steps = np.concatenate([dct_host.steps(q, m.dct["dc_step"]).reshape(-1) for q in m.dct["q"]])
        tr.set_dct(d, m.dct["code"], m.dct["sym"], steps)
    return tr


def load(path: str) -> model_file.ModelFile:
    """a model file or a container (told apart by the magic), as the model the decode needs"""
    with open(path, "rb") as f:
        head = f.read(4)
    if len(head) == 4 and struct.unpack("<I", head)[0] == ntcb.MAGIC:
        return ntcb.read(path).to_model_file()
    return model_file.read(path)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("model")
    ap.add_argument("out_prefix", nargs="?", default="")
    ap.add_argument("--repeat", type=int, default=0, help="time this many decodes and report Mtexel/s")
    a = ap.parse_args(argv)
    m = load(a.model)
    lay = m.layout
    tr = trainer_for(m)
    rgb = tr.decode_rgb8().reshape(lay.H, lay.W, lay.nout)
    sw, sh = (m.size[2], m.size[3]) if m.size[2] > 0 else (lay.W, lay.H)
    if a.out_prefix:
        for t in range(lay.T):
            name = f"{a.out_prefix}.png" if lay.T == 1 else f"{a.out_prefix}_t{t}.png"
            write_png(name, np.ascontiguousarray(rgb[:sh, :sw, 3 * t:3 * t + 3]))
    if a.repeat > 0:
        tr.synchronize()
        tr.set_profiling(True)
        t0 = time.perf_counter()
        for _ in range(a.repeat):
            tr.decode_rgb8()
        el = time.perf_counter() - t0
        dk, n = tr.kernel_time("decode")
        pk, _ = tr.kernel_time("pack_u8")
        texels = lay.W * lay.H
        print(json.dumps({"model": a.model, "texels": texels, "textures": lay.T, "mlp": [lay.nin] + list(lay.hidden) + [lay.nout],
                          "device_ms": (dk + pk) / n, "device_mtexel_s": texels / ((dk + pk) / n * 1e-3) / 1e6,
                          "with_download_ms": 1e3 * el / a.repeat, "with_download_mtexel_s": texels * a.repeat / el / 1e6}))
    tr.close()


if __name__ == "__main__":
    sys.exit(main())
