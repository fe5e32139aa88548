"""The reference's model files (main.cpp save_model 2156-2210, the loader 3567-3700): v9 .. v14.

A model file is little-endian ints and floats:
  int hdr[10]   magic, level-0 W H C, nin, spec length, activation (0), hidden layers, levels, textures
  int filter[levels]                    0 bilinear, 1 nearest
  int deblock, float falloff            layout only (deblock must be 0)
  float leak                            (v8+)
  int qat                               largest --qat bit depth (v9+)
  int qat_ch[C0]                        (v10+)
  int W, H, orig_w, orig_h, clamp       (v11+)
  int dims[levels - 1][3]               W, H, C of levels 1..
  per level: int qes_bits, float lo[C], float hi[C]      (v12+)
  int dct_N, dct_dc_step, dct_C [, dct_deadzone (v14)], int q[dct_C]   (v13+, DCT-coded level 0)
  int hidden[layers], char spec[len]
  payload: the flat latent (levels concatenated, (y, x, c)), or - in a DCT file - int16 symbols
  [blocks][C][64], uint8 codes [blocks][C] and the floats of levels >= 1; then the MLP parameters.

Magics: v9 0x4E544339 .. v12 0x4E54433C, v13 0x4E54433D, v14 0x4E54433E.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

from .trainer import PK_LV1LOCAL, PK_UV, Layout

MAGIC = {0x4E544339: 9, 0x4E54433A: 10, 0x4E54433B: 11, 0x4E54433C: 12, 0x4E54433D: 13, 0x4E54433E: 14}
MAGIC_OF = {v: k for k, v in MAGIC.items()}


@dataclass
class ModelFile:
    version: int
    layout: Layout
    z: np.ndarray                     # the flat latent (level 0 left zero in a DCT file: its plane comes from the symbols)
    p: np.ndarray                     # MLP parameters
    qat: int = 0
    qat_ch: list = field(default_factory=list)
    clamp: bool = False
    size: tuple = (0, 0, 0, 0)        # decoded W, H, source W, H
    qes: list = field(default_factory=list)   # per level (bits, lo[C], hi[C])
    dct: dict | None = None           # {"N", "dc_step", "deadzone", "q": [C], "sym": int16, "code": uint8}


def _pos_kinds(spec: str) -> list:
    if spec in ("", "none"):
        return []
    kinds = {"uv": PK_UV, "lv1local": PK_LV1LOCAL}
    return [kinds[s] for s in spec.split(",")]


def _spec(kinds) -> str:
    names = {PK_UV: "uv", PK_LV1LOCAL: "lv1local"}
    return ",".join(names[k] for k in kinds)


def read(path: str) -> ModelFile:
    with open(path, "rb") as f:
        b = f.read()
    o = 0

    def ints(n):
        nonlocal o
        if o + 4 * n > len(b):
            raise ValueError(f"{path}: truncated")
        v = struct.unpack_from(f"<{n}i", b, o)
        o += 4 * n
        return list(v)

    def f32(n):
        nonlocal o
        if o + 4 * n > len(b):
            raise ValueError(f"{path}: truncated")
        v = np.frombuffer(b, np.float32, n, o).copy()
        o += 4 * n
        return v

    hdr = ints(10)
    magic = hdr[0] & 0xFFFFFFFF
    if magic not in MAGIC:
        raise ValueError(f"{path}: not a v9..v14 ntc model file")
    ver = MAGIC[magic]
    _, LW0, LH0, LC0, nin, poslen, act, nl, nlev, T = hdr
    if act != 0:
        raise ValueError(f"{path}: saved with activation {act}; only leaky is supported")
    if not (1 <= nl <= 8 and 1 <= nlev <= 3 and 1 <= T <= 4):
        raise ValueError(f"{path}: corrupt header")
    filt = ints(nlev)
    deblock = ints(1)[0]
    f32(1)                                           # falloff: layout only
    if deblock != 0:
        raise ValueError(f"{path}: deblocking is not supported")
    leak = float(f32(1)[0])
    qat = ints(1)[0]
    qat_ch = ints(LC0) if ver >= 10 else [qat] * LC0
    size, clamp = (0, 0, 0, 0), False
    if ver >= 11:
        img = ints(5)
        size, clamp = tuple(img[:4]), img[4] == 1
    dims = [(LW0, LH0, LC0)] + [tuple(ints(3)) for _ in range(nlev - 1)]
    qes = []
    if ver >= 12:
        for l in range(nlev):
            bits = ints(1)[0]
            qes.append((bits, f32(dims[l][2]), f32(dims[l][2])))
    dct = None
    if ver >= 13:
        N, dc_step, C = ints(3)
        dz = ints(1)[0] if ver >= 14 else 1
        dct = {"N": N, "dc_step": dc_step, "deadzone": dz, "q": ints(C)}
        if N != 8 or C != LC0 or LW0 % 8 or LH0 % 8 or filt[0] != 1:
            raise ValueError(f"{path}: bad DCT header")
    hidden = ints(nl)
    spec = b[o:o + poslen].decode()
    o += poslen
    W, H = (size[0], size[1]) if ver >= 11 else (0, 0)
    lay = Layout(W, H, [(w, h, c, filt[l] == 1) for l, (w, h, c) in enumerate(dims)], hidden, T=T, pos=_pos_kinds(spec),
                 leak=leak, clamp_out=clamp)
    if lay.nin != nin:
        raise ValueError(f"{path}: nin {nin} does not match the levels and the positional spec")
    nz = sum(w * h * c for w, h, c in dims)
    if dct is not None:
        nb = (LW0 // 8) * (LH0 // 8)
        if o + nb * LC0 * 64 * 2 + nb * LC0 > len(b):
            raise ValueError(f"{path}: truncated")
        dct["sym"] = np.frombuffer(b, np.int16, nb * LC0 * 64, o).copy()
        o += nb * LC0 * 64 * 2
        dct["code"] = np.frombuffer(b, np.uint8, nb * LC0, o).copy()
        o += nb * LC0
        n0 = LW0 * LH0 * LC0
        z = np.zeros(nz, np.float32)
        z[n0:] = f32(nz - n0)
    else:
        z = f32(nz)
    p = f32(lay.nparams)
    if o != len(b):
        raise ValueError(f"{path}: {len(b) - o} trailing bytes")
    return ModelFile(ver, lay, z, p, qat, qat_ch, clamp, size, qes, dct)


def write(path: str, m: ModelFile) -> None:
    """save_model's layout: v12, or v14 when m.dct is set (the version field is ignored)"""
    lay = m.layout
    dct = m.dct
    W0, H0, C0, _ = lay.levels[0]
    out = [struct.pack("<10i", MAGIC_OF[14 if dct else 12], W0, H0, C0, lay.nin, len(_spec(lay.pos)), 0, len(lay.hidden),
                       len(lay.levels), lay.T)]
    out += [struct.pack("<i", 1 if nr else 0) for (_, _, _, nr) in lay.levels]
    out += [struct.pack("<if", 0, 1.0), struct.pack("<f", lay.leak), struct.pack("<i", m.qat)]
    qch = list(m.qat_ch) or [0] * C0
    out += [struct.pack(f"<{C0}i", *qch)]
    sz = m.size if any(m.size) else (lay.W, lay.H, lay.W, lay.H)
    out += [struct.pack("<5i", *sz, 1 if lay.clamp_out else 0)]
    out += [struct.pack("<3i", w, h, c) for (w, h, c, _) in lay.levels[1:]]
    for l, (w, h, c, _) in enumerate(lay.levels):
        bits, lo, hi = m.qes[l] if m.qes else (0, np.zeros(c, np.float32), np.zeros(c, np.float32))
        out += [struct.pack("<i", bits), np.asarray(lo, np.float32).tobytes(), np.asarray(hi, np.float32).tobytes()]
    if dct:
        out += [struct.pack("<4i", 8, dct["dc_step"], C0, dct["deadzone"]), struct.pack(f"<{C0}i", *dct["q"])]
    out += [struct.pack(f"<{len(lay.hidden)}i", *lay.hidden), _spec(lay.pos).encode()]
    if dct:
        n0 = W0 * H0 * C0
        out += [np.asarray(dct["sym"], np.int16).tobytes(), np.asarray(dct["code"], np.uint8).tobytes(),
                np.asarray(m.z[n0:], np.float32).tobytes()]
    else:
        out += [np.asarray(m.z, np.float32).tobytes()]
    out += [np.asarray(m.p, np.float32).tobytes()]
    with open(path, "wb") as f:
        f.write(b"".join(out))
