"""Decode a model file of the reference (model.bin v11 .. v14, or the bit-packed model.ntcb) on the GPU
to 8-bit PNGs, one per texture, cropped to the source extent the file records (as ntc_decode writes).

    python -m neural_block_textures_amd.decode model.bin|model.ntcb out_prefix [--fp32-latent | --q8]
        [--no-crop | --crop W H] [--compare PNG[,PNG...]] [--repeat 50]

As ntc_decode (ntc_decode.cpp:1210-1230, 322-342), a model file's levels that training left continuous are
decoded on bitrate_stats' post-hoc 8-bit grid by default (--q8; the values recon_q_final.png shows), or
as stored with --fp32-latent (recon_NNNNNN.png); --qat, --qes and DCT levels are used as stored, and a
container holds grid indices already.

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


def level_quantized(m: model_file.ModelFile, l: int) -> bool:
    """a level training kept on a grid: a --qat or DCT-coded level 0, or a --qes level"""
    return (l == 0 and (m.qat > 0 or m.dct is not None)) or (bool(m.qes) and m.qes[l][0] > 0)


def q8_quantize(m: model_file.ModelFile, qbits: int = 8) -> None:
    """bitrate_stats' post-hoc quantization of the continuous levels, in place (per channel min / max
    grid, lround index, strict float32 values; main.cpp:2273-2352, ntc_decode.cpp:324-342)"""
    lay = m.layout
    levels = (1 << qbits) - 1
    for l, ((W, H, C, _), off) in enumerate(zip(lay.levels, lay.offsets)):
        if level_quantized(m, l):
            continue
        z = m.z[off:off + W * H * C].reshape(-1, C)
        for c in range(C):
            lo, hi = np.float32(z[:, c].min()), np.float32(z[:, c].max())
            rng = max(np.float32(hi - lo), np.float32(1e-6))
            z[:, c] = ntcb.grid_values(lo, hi, qbits)[ntcb.q8_index(z[:, c], lo, rng, levels)]


def load(path: str, q8: bool = True) -> model_file.ModelFile:
    """a model file or a container (told apart by the magic), as the model the decode needs; a model
    file's continuous levels on the post-hoc 8-bit grid unless q8 is False"""
    with open(path, "rb") as f:
        head = f.read(4)
    if len(head) == 4 and struct.unpack("<I", head)[0] == ntcb.MAGIC:
        return ntcb.read(path).to_model_file()
    m = model_file.read(path)
    if q8:
        q8_quantize(m)
    return m


def read_png(path: str) -> np.ndarray:
    """an 8-bit RGB(A) PNG as H x W x 3 (for --compare)"""
    try:
        from PIL import Image
    except ImportError as e:   # the comparison is optional; the decode itself needs nothing
        raise SystemExit(f"--compare needs PIL to read {path}: {e}")
    return np.asarray(Image.open(path).convert("RGB"))


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("model")
    ap.add_argument("out_prefix", nargs="?", default="")
    ap.add_argument("--repeat", type=int, default=0, help="time this many decodes and report Mtexel/s")
    q = ap.add_mutually_exclusive_group()
    q.add_argument("--fp32-latent", action="store_true", help="decode the stored latent values as they are")
    q.add_argument("--q8", action="store_true", help="post-hoc 8-bit grid for the continuous levels (default)")
    cr = ap.add_mutually_exclusive_group()
    cr.add_argument("--no-crop", action="store_true", help="write the full decoded (padded) image")
    cr.add_argument("--crop", type=int, nargs=2, metavar=("W", "H"), help="write only the top-left W x H")
    ap.add_argument("--compare", help="per-texture reference PNGs, comma-separated: PSNR and max |diff|")
    a = ap.parse_args(argv)
    m = load(a.model, q8=not a.fp32_latent)
    lay = m.layout
    tr = trainer_for(m)
    rgb = tr.decode_rgb8().reshape(lay.H, lay.W, lay.nout)
    sw, sh = (m.size[2], m.size[3]) if m.size[2] > 0 else (lay.W, lay.H)
    if a.no_crop:
        sw, sh = lay.W, lay.H
    elif a.crop:
        sw, sh = a.crop
        if sw > lay.W or sh > lay.H or sw < 1 or sh < 1:
            raise SystemExit(f"--crop {sw}x{sh} exceeds the decode size {lay.W}x{lay.H}")
    if a.compare:
        refs = a.compare.split(",")
        if len(refs) != lay.T:
            raise SystemExit(f"--compare needs {lay.T} PNG(s), got {len(refs)}")
        for t, ref in enumerate(refs):
            r = read_png(ref).astype(np.int64)
            d = rgb[:sh, :sw, 3 * t:3 * t + 3].astype(np.int64)
            if r.shape != d.shape:
                raise SystemExit(f"{ref}: {r.shape[1]}x{r.shape[0]}, the decode is {sw}x{sh}")
            diff = np.abs(d - r)
            mse = float((diff ** 2).mean())
            psnr = 100.0 if mse == 0 else 10.0 * np.log10(255.0 ** 2 / mse)
            print(json.dumps({"compare": ref, "texture": t, "psnr_db": round(psnr, 2), "max_abs_diff": int(diff.max()),
                              "equal_fraction": float((diff == 0).mean())}))
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
