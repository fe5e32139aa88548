"""The reference's bit-packed model container, model.ntcb (main.cpp:2355-2846, the NTCB region; its
standalone decoder's load_ntcb in ntc_decode.cpp): read and validate, write, and hand the model to
the GPU decode.

Layout (every field little-endian; version 2, version 1 also read):
  header, H bytes
    u32 magic "ntcb" (0x6263746E), u16 version, u16 H, u32 img_w img_h src_w src_h,
    u32 file_bytes, u32 hash (FNV-1a 32 of the whole file with these four bytes read as zero),
    u8 latent_cell dct_block T nlevels act(0) clamp nhidden reserved(0), f32 leak, u32 nin nout,
    u8 channels[T] (3 each), u16 hidden[nhidden], u16 len + the positional spec text,
    per level: u32 W H, u16 C, u8 filter (1 nearest), u8 mode, u8 bits[C], then
      mode 0 (post-hoc grid) / 1 (--qes grid): f32 lo hi per channel,
      mode 2 (--qat palette): f32 palette[C][2^bits],
      mode 3 (--dct-q, level 0 only): u8 dc_step, u8 dct_flags (version 2; bit 0 = dead zone), u8 q[C]
  sections: an 8-byte record (u8 kind (1 level, 2 MLP), u8 coding 0, u8 level, u8 0, u32 length)
  and an LSB-first bit stream padded with zeros to the byte:
    level l: sync(LEVEL, l), [mode 3: per channel sync(CHANNEL, l, c), the 4-bit scale codes of
      every block, then per block the DC symbol (dc_raw_bits) and the AC tokens in zigzag order
      (run 7 bits, |q| - 1 8 bits, sign 1 bit), EOB (run 64) unless position 63 is nonzero]
      [modes 0-2: per channel, per texel in (y, x) order: the grid index, bits[c] wide],
      sync(END, l)
    MLP: sync(MLP, nlevels), the fp16 weights in parameter order, sync(END, nlevels)
  A sync marker is 6 bits: (base + 13 level + 7 channel) & 63.

A grid level's values are lo + k / (float)levels * range with range = max(hi - lo, 1e-6f), in
float32 (qes_rebuild, main.cpp:466-476); a palette level's are the stored floats; the weights are
the fp16 values widened.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

from . import dct_host
from .model_file import ModelFile, _pos_kinds, _spec
from .trainer import Layout

MAGIC = 0x6263746E
VERSION = 2
FIXED_HEADER = 52
SYNC_LEVEL, SYNC_CHANNEL, SYNC_MLP, SYNC_END, SYNC_BITS = 0x2B, 0x16, 0x31, 0x0C, 6
DCT_EOB = 64
MAX_T, MAX_L, MAX_H, MAX_DCT_CH = 4, 8, 64, 4


def sync_value(base: int, level: int, channel: int = 0) -> int:
    return (base + 13 * level + 7 * channel) & 63


def file_hash(b: bytes) -> int:
    """FNV-1a 32 over the file with bytes 28..31 (the hash field) read as zero"""
    h = 2166136261
    for i, v in enumerate(b):
        h = ((h ^ (0 if 28 <= i < 32 else v)) * 16777619) & 0xFFFFFFFF
    return h


def dc_raw_bits(dc_step: int) -> int:
    """ceil(log2(floor(512 / dc_step) + 1)): the fixed width of a DC symbol"""
    lvl, b = 512 // dc_step + 1, 0
    while (1 << b) < lvl:
        b += 1
    return b


def f16_bits(p: np.ndarray) -> np.ndarray:
    """the fp16 patterns of weights that are fp16 values; ValueError otherwise (the writer never rounds)"""
    p = np.asarray(p, np.float32)
    if not np.isfinite(p).all():
        raise ValueError("a weight is not finite")
    with np.errstate(over="ignore"):
        h = p.astype(np.float16)
    if not np.isfinite(h).all():
        raise ValueError("a weight is above the fp16 range")
    if not np.array_equal(h.astype(np.float32), p):
        i = int(np.nonzero(h.astype(np.float32) != p)[0][0])
        raise ValueError(f"weight {i} = {p[i]!r} is not an fp16 value (round the weights first)")
    return h.view(np.uint16)


def round_fp16(p: np.ndarray) -> np.ndarray:
    """ntcb_mlp_round_fp16 (main.cpp:2472-2481): every weight rounded to the nearest fp16 value"""
    p = np.asarray(p, np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        h = p.astype(np.float16)
    if not np.isfinite(p).all() or not np.isfinite(h).all():
        raise ValueError("a weight is non-finite or above 65504 and has no fp16 value")
    return h.astype(np.float32)


# ---- the grids (strict float32, as the reference's STRICT_FP region computes them)

def grid_values(lo: float, hi: float, bits: int) -> np.ndarray:
    """qes_rebuild: lo + k / (float)levels * range, range = max(hi - lo, 1e-6f)"""
    levels = (1 << bits) - 1
    lo, hi = np.float32(lo), np.float32(hi)
    rng = max(np.float32(hi - lo), np.float32(1e-6))
    k = np.arange(levels + 1, dtype=np.float32)
    return (lo + (k / np.float32(levels)) * rng).astype(np.float32)


def q8_index(z: np.ndarray, lo, rng, levels: int) -> np.ndarray:
    """q8_index (main.cpp:478-481): lround((z - lo) / range * levels), clamped"""
    x = ((np.asarray(z, np.float32) - np.float32(lo)) / np.float32(rng) * np.float32(levels)).astype(np.float64)
    k = np.floor(np.abs(x) + 0.5) * np.sign(x)
    return np.clip(k, 0, levels).astype(np.int64)


def qes_index(z: np.ndarray, lo, rng, levels: int) -> np.ndarray:
    """qes_index (main.cpp:448-453): round-half-even of ((v - lo) / range) * levels, clamped in float"""
    r = np.rint(((np.asarray(z, np.float32) - np.float32(lo)) / np.float32(rng)) * np.float32(levels))
    return np.clip(r, 0, levels).astype(np.int64)


def qat_palette(bits: int) -> np.ndarray:
    """QAT_GRID[bits] (main.cpp:2054-2057): -1 + 2 k / levels in float"""
    levels = (1 << bits) - 1
    k = np.arange(levels + 1, dtype=np.float32)
    return (np.float32(-1.0) + (np.float32(2.0) * k) / np.float32(levels)).astype(np.float32)


def qat_index(z: np.ndarray, bits: int) -> np.ndarray:
    """qat_index (main.cpp:2060-2064): lround((v + 1) * 0.5 * levels), clamped"""
    levels = (1 << bits) - 1
    x = ((np.asarray(z, np.float32) + np.float32(1.0)) * np.float32(0.5) * np.float32(levels)).astype(np.float64)
    return np.clip(np.floor(np.abs(x) + 0.5) * np.sign(x), 0, levels).astype(np.int64)


# ---- bit streams (LSB first)

class _Bits:
    """a bit stream under construction: chunks of 0/1 bytes, packed LSB-first at the end"""

    def __init__(self):
        self.chunks, self.n, self.sync = [], 0, 0

    def put(self, v, width: int):
        """one value, or an array of values, each `width` bits"""
        v = np.atleast_1d(np.asarray(v, np.int64))
        self.chunks.append(((v[:, None] >> np.arange(width)) & 1).astype(np.uint8).reshape(-1))
        self.n += width * v.size

    def marker(self, m: int):
        self.put(m, SYNC_BITS)
        self.sync += SYNC_BITS

    def bytes(self) -> bytes:
        bits = np.concatenate(self.chunks) if self.chunks else np.zeros(0, np.uint8)
        return np.packbits(bits, bitorder="little").tobytes()


class _Reader:
    """the bits of one section, read LSB-first; `fail` names what ran past the end"""

    def __init__(self, body: bytes):
        self.bits = np.unpackbits(np.frombuffer(body, np.uint8), bitorder="little")
        self.pos = 0

    def get(self, width: int, count: int = 1, what: str = "") -> np.ndarray:
        end = self.pos + width * count
        if end > self.bits.size:
            raise ValueError(f"truncated {what}".strip())
        v = self.bits[self.pos:end].reshape(count, width).astype(np.int64) @ (np.int64(1) << np.arange(width, dtype=np.int64))
        self.pos = end
        return v

    def get1(self, width: int, what: str = "") -> int:
        return int(self.get(width, 1, what)[0])

    def marker(self, m: int, where: str):
        if self.pos + SYNC_BITS > self.bits.size or self.get1(SYNC_BITS) != m:
            raise ValueError(f"sync marker mismatch {where}")

    def aligned_bytes(self) -> int:
        return (self.pos + 7) // 8


# ---- the container

@dataclass
class NtcbLevel:
    W: int
    H: int
    C: int
    nearest: bool
    mode: int                       # 0 post-hoc grid, 1 --qes grid, 2 --qat palette, 3 DCT
    bits: list                      # per channel (0 for mode 3)
    lo: np.ndarray | None = None    # modes 0 / 1
    hi: np.ndarray | None = None
    palette: list | None = None     # mode 2: per channel 2^bits floats
    dc_step: int = 0                # mode 3
    deadzone: int = 1
    q: list = field(default_factory=list)
    idx: np.ndarray | None = None   # modes 0-2: grid indices, (y, x, c) with c fastest
    sym: np.ndarray | None = None   # mode 3: int16 [blocks][C][64], natural order
    code: np.ndarray | None = None  # mode 3: uint8 [blocks][C]

    def values(self) -> np.ndarray:
        """the level's decode values, (y, x, c) with c fastest (zeros for a DCT level: its plane is
        reconstructed from the symbols)"""
        n = self.W * self.H * self.C
        if self.mode == 3:
            return np.zeros(n, np.float32)
        out = np.empty(n, np.float32)
        for c in range(self.C):
            table = self.palette[c] if self.mode == 2 else grid_values(self.lo[c], self.hi[c], self.bits[c])
            out[c::self.C] = table[self.idx[c::self.C]]
        return out


@dataclass
class Ntcb:
    img_w: int
    img_h: int
    src_w: int
    src_h: int
    levels: list
    hidden: list
    p: np.ndarray                   # the MLP parameters (fp16 values)
    T: int = 1
    leak: float = 0.01
    clamp: bool = False
    pos: str = "uv"
    latent_cell: int = 0
    version: int = VERSION

    @property
    def dct_block(self) -> int:
        return 8 if self.levels and self.levels[0].mode == 3 else 0

    @property
    def layout(self) -> Layout:
        return Layout(self.img_w, self.img_h, [(L.W, L.H, L.C, L.nearest) for L in self.levels], list(self.hidden), T=self.T,
                      pos=_pos_kinds(self.pos), leak=float(self.leak), clamp_out=bool(self.clamp))

    def to_model_file(self) -> ModelFile:
        """the model as the reference's loader installs it (ntcb_restore): decode values of every level,
        a --qat level 0 with its bit depths, --qes levels with their grids, a DCT level 0's symbols"""
        lay = self.layout
        z = np.concatenate([L.values() for L in self.levels])
        L0 = self.levels[0]
        qat_ch = list(L0.bits) if L0.mode == 2 else []
        qes = [(L.bits[0], np.asarray(L.lo, np.float32), np.asarray(L.hi, np.float32)) if L.mode == 1
               else (0, np.zeros(L.C, np.float32), np.zeros(L.C, np.float32)) for L in self.levels]
        dct = None
        if L0.mode == 3:
            dct = {"N": 8, "dc_step": L0.dc_step, "deadzone": L0.deadzone, "q": list(L0.q), "sym": L0.sym.copy(), "code": L0.code.copy()}
        return ModelFile(14 if dct else 12, lay, z, np.asarray(self.p, np.float32).copy(), max(qat_ch) if qat_ch else 0, qat_ch,
                         bool(self.clamp), (self.img_w, self.img_h, self.src_w, self.src_h), qes, dct)


def _header(n: Ntcb) -> bytearray:
    """ntcb_write_header (main.cpp:2500-2522); H patched in, file_bytes and hash left zero"""
    lay = n.layout
    b = bytearray(struct.pack("<IHH4III", MAGIC, n.version, 0, n.img_w, n.img_h, n.src_w, n.src_h, 0, 0))
    b += struct.pack("<8B", n.latent_cell, n.dct_block, n.T, len(n.levels), 0, 1 if n.clamp else 0, len(n.hidden), 0)
    b += struct.pack("<fII", n.leak, lay.nin, lay.nout)
    b += bytes([3] * n.T)
    b += struct.pack(f"<{len(n.hidden)}H", *n.hidden)
    b += struct.pack("<H", len(n.pos)) + n.pos.encode()
    for L in n.levels:
        b += struct.pack("<IIHBB", L.W, L.H, L.C, 1 if L.nearest else 0, L.mode) + bytes(L.bits)
        if L.mode == 3:
            b += bytes([L.dc_step] + ([1 if L.deadzone else 0] if n.version >= 2 else []) + list(L.q))
        if L.mode in (0, 1):
            for c in range(L.C):
                b += struct.pack("<ff", float(np.float32(L.lo[c])), float(np.float32(L.hi[c])))
        if L.mode == 2:
            for c in range(L.C):
                b += np.asarray(L.palette[c], np.float32).tobytes()
    if len(b) > 65535:
        raise ValueError("header larger than 65535 bytes")
    struct.pack_into("<H", b, 6, len(b))
    return b


def _level_bits(n: Ntcb, l: int) -> _Bits:
    L = n.levels[l]
    w = _Bits()
    w.marker(sync_value(SYNC_LEVEL, l))
    if L.mode == 3:
        zz = dct_host.zigzag()
        drb = dc_raw_bits(L.dc_step)
        nb = (L.W // 8) * (L.H // 8)
        sym = np.asarray(L.sym, np.int16).reshape(nb, L.C, 64)
        code = np.asarray(L.code, np.uint8).reshape(nb, L.C)
        for c in range(L.C):
            w.marker(sync_value(SYNC_CHANNEL, l, c))
            w.put(code[:, c], 4)
            vals, widths = [], []
            for b in range(nb):
                s = sym[b, c]
                if s[0] < 0 or s[0] >= (1 << drb):
                    raise ValueError(f"DC symbol {int(s[0])} of block {b}, channel {c} does not fit {drb} unsigned bits")
                vals.append(int(s[0])); widths.append(drb)
                run, lnz = 0, 0
                for p in range(1, 64):
                    q = int(s[zz[p]])
                    if q == 0:
                        run += 1
                        continue
                    if abs(q) > 256:
                        raise ValueError(f"|q| = {abs(q)} > 256 at block {b}, channel {c}")
                    vals += [run, abs(q) - 1, 1 if q < 0 else 0]; widths += [7, 8, 1]
                    lnz, run = p, 0
                if lnz < 63:
                    vals.append(DCT_EOB); widths.append(7)
            # the block stream as one bit array: each value expanded to its own width
            v = np.asarray(vals, np.int64); wd = np.asarray(widths, np.int64)
            starts = np.repeat(np.cumsum(wd) - wd, wd)
            shift = np.arange(int(wd.sum())) - starts
            w.chunks.append(((np.repeat(v, wd) >> shift) & 1).astype(np.uint8))
            w.n += int(wd.sum())
    else:
        for c in range(L.C):
            w.put(np.asarray(L.idx, np.int64)[c::L.C], L.bits[c])
    w.marker(sync_value(SYNC_END, l))
    return w


def to_bytes(n: Ntcb) -> bytes:
    """the file ntcb_write (main.cpp:2637-2755) writes for this content"""
    out = _header(n)
    for l in range(len(n.levels)):
        body = _level_bits(n, l).bytes()
        out += struct.pack("<BBBBI", 1, 0, l, 0, len(body)) + body
    w = _Bits()
    w.marker(sync_value(SYNC_MLP, len(n.levels)))
    w.put(f16_bits(n.p), 16)
    w.marker(sync_value(SYNC_END, len(n.levels)))
    body = w.bytes()
    out += struct.pack("<BBBBI", 2, 0, 0, 0, len(body)) + body
    struct.pack_into("<I", out, 24, len(out))
    struct.pack_into("<I", out, 28, file_hash(bytes(out)))
    return bytes(out)


def write(path: str, n: Ntcb) -> int:
    b = to_bytes(n)
    with open(path, "wb") as f:
        f.write(b)
    return len(b)


def _min_section_bytes(img_levels: list, nin: int, hidden: list, nout: int) -> int:
    """ntcb_min_section_bytes (main.cpp:2524-2538)"""
    total = 0
    for L in img_levels:
        bits = 2 * SYNC_BITS
        if L.mode == 3:
            nblk = (L.W // 8) * (L.H // 8)
            bits += L.C * (SYNC_BITS + nblk * (4 + dc_raw_bits(L.dc_step) + 7))
        else:
            bits += sum(L.W * L.H * b for b in L.bits)
        total += 8 + (bits + 7) // 8
    nparams, prev = 0, nin
    for w in hidden:
        nparams += w * prev + w
        prev = w
    nparams += nout * prev + nout
    return total + 8 + (16 * nparams + 2 * SYNC_BITS + 7) // 8


def parse(buf: bytes) -> Ntcb:
    """ntcb_read_header + ntcb_restore (main.cpp:2540-2618, 2762-2846): every check, in the same
    order, raising ValueError with the reason"""
    n = len(buf)
    if n < 8:
        raise ValueError("not an ntcb file (shorter than 8 bytes)")
    magic, version, H = struct.unpack_from("<IHH", buf, 0)
    if magic != MAGIC:
        raise ValueError("not an ntcb file (bad magic)")
    if version not in (1, VERSION):
        raise ValueError(f"ntcb version {version} (this build reads versions 1 and {VERSION})")
    if H < FIXED_HEADER or H > n:
        raise ValueError(f"header length {H} exceeds the file size {n} (truncated or corrupt)")
    hb = buf[:H]
    o = 8

    def take(fmt):
        nonlocal o
        size = struct.calcsize(fmt)
        if o + size > H:
            raise ValueError("truncated header")
        v = struct.unpack_from(fmt, hb, o)
        o += size
        return v

    img_w, img_h, src_w, src_h, file_bytes, hsh = take("<6I")
    if file_bytes != n:
        raise ValueError(f"file_bytes {file_bytes} != actual size {n} (truncated or extended)")
    if file_hash(buf) != hsh:
        raise ValueError("file hash mismatch (corrupt file)")
    latent_cell, dct_block, T, nlevels, act, clamp, nhidden, reserved = take("<8B")
    leak, nin, nout = take("<fII")
    if not (1 <= img_w <= 16384 and 1 <= img_h <= 16384 and 1 <= src_w <= img_w and 1 <= src_h <= img_h):
        raise ValueError("bad image size fields (decode size at most 16384 x 16384, source size within it)")
    if not (1 <= T <= MAX_T and 1 <= nlevels <= 3 and act == 0 and clamp in (0, 1) and 1 <= nhidden <= MAX_L and reserved == 0):
        raise ValueError("header field out of range (textures 1..4, 1..3 levels, activation 0, clamp 0/1, 1..8 hidden layers, reserved byte 0)")
    if not np.isfinite(np.float32(leak)) or not (1 <= nin <= MAX_H) or not (1 <= nout <= MAX_H):
        raise ValueError("bad leak, nin or nout")
    cpt = take(f"<{T}B")
    for t, c in enumerate(cpt):
        if c != 3:
            raise ValueError(f"texture {t} has {c} channels; this build decodes 3 per texture")
    if sum(cpt) != nout:
        raise ValueError(f"nout {nout} != the sum of the per-texture channel counts {sum(cpt)}")
    hidden = list(take(f"<{nhidden}H"))
    if any(not (1 <= w <= MAX_H) for w in hidden):
        raise ValueError("bad hidden width")
    (poslen,) = take("<H")
    if poslen >= 4096:
        raise ValueError("bad positional spec length")
    if o + poslen > H:
        raise ValueError("truncated header (positional spec)")
    pos = hb[o:o + poslen].decode("latin-1")
    o += poslen
    levels, chsum = [], 0
    for l in range(nlevels):
        lv = f"level {l}: "
        try:
            W, Hh, C, filt, mode = take("<IIHBB")
        except ValueError:
            raise ValueError(lv + "truncated level record") from None
        if not (1 <= W <= (1 << 20) and 1 <= Hh <= (1 << 20) and 1 <= C <= MAX_H and filt in (0, 1) and 0 <= mode <= 3):
            raise ValueError(lv + f"bad dims ({W}x{Hh}x{C}), filter flag ({filt}) or mode ({mode})")
        if l > 0 and mode > 1:
            raise ValueError(lv + f"mode {mode} (qat / dct) is only defined on level 0")
        try:
            bits = list(take(f"<{C}B"))
        except ValueError:
            raise ValueError(lv + "truncated level record") from None
        for B in bits:
            ok = B == 0 if mode == 3 else ((1 <= B <= 8) if mode == 2 else (2 <= B <= 12))
            if not ok:
                raise ValueError(lv + f"bit depth {B} out of range for mode {mode}")
            if mode <= 1 and B != bits[0]:
                raise ValueError(lv + "per-channel bit depths on a grid level are not supported by this trainer")
        L = NtcbLevel(W, Hh, C, filt == 1, mode, bits)
        if mode == 3:
            try:
                (L.dc_step,) = take("<B")
                flags = take("<B")[0] if version >= 2 else 1
                L.q = list(take(f"<{C}B"))
            except ValueError:
                raise ValueError(lv + "truncated level record") from None
            if not 1 <= L.dc_step <= 64:
                raise ValueError(lv + f"dc_step {L.dc_step} out of range (1..64)")
            if flags & ~1:
                raise ValueError(lv + f"dct_flags {flags} has reserved bits set (only bit 0, the dead zone, is defined)")
            L.deadzone = flags & 1
            for q in L.q:
                if not 1 <= q <= 100:
                    raise ValueError(lv + f"dct quality {q} out of range (1..100)")
            if dct_block != 8 or filt != 1 or W != img_w or Hh != img_h or W % 8 or Hh % 8 or C > MAX_DCT_CH:
                raise ValueError(lv + "a dct level must be a full-resolution nearest level with a size that is a multiple of 8, "
                                 "dct_block 8 and at most 4 channels")
        elif l == 0 and dct_block != 0:
            raise ValueError("dct_block must be 0 when level 0 is not DCT-coded")
        if mode == 2 and filt != 1:
            raise ValueError(lv + "a qat level must be nearest")
        if mode <= 1:
            try:
                r = np.array(take(f"<{2 * C}f"), np.float32).reshape(C, 2)
            except ValueError:
                raise ValueError(lv + "truncated grid ranges") from None
            L.lo, L.hi = r[:, 0].copy(), r[:, 1].copy()
            if not (np.isfinite(r).all() and (L.lo <= L.hi).all()):
                raise ValueError(lv + "bad grid range")
        if mode == 2:
            L.palette = []
            for c in range(C):
                try:
                    pal = np.array(take(f"<{1 << bits[c]}f"), np.float32)
                except ValueError:
                    raise ValueError(lv + "truncated palette") from None
                if not np.isfinite(pal).all():
                    raise ValueError(lv + "non-finite palette value")
                L.palette.append(pal)
        chsum += C
        levels.append(L)
    if o != H:
        raise ValueError(f"header length {H} disagrees with its fields ({o} bytes)")
    kinds = {"uv", "lv1local"}
    if pos not in ("", "none") and any(s not in kinds for s in pos.split(",")):
        raise ValueError(f'positional spec "{pos}" is not one this build reads')
    npos = 0 if pos in ("", "none") else 2 * len(pos.split(","))
    if chsum + npos != nin:
        raise ValueError(f"nin {nin} != latent channels {chsum} + positional inputs {npos}")
    need = _min_section_bytes(levels, nin, hidden, nout)
    if need > n - H:
        raise ValueError(f"the header's sections need at least {need} bytes but the file has {n - H} after the header (truncated or corrupt)")

    # the sections
    pos_b = H
    zz = dct_host.zigzag()

    def section(kind, level):
        nonlocal pos_b
        name = f"level {level}" if kind == 1 else "the mlp"
        if pos_b + 8 > n:
            raise ValueError(f"truncated at the section header of {name}")
        k, coding, lv, res, ln = struct.unpack_from("<BBBBI", buf, pos_b)
        if coding != 0:
            raise ValueError(f"coded sections (coding {coding}) need a newer decoder" if coding in (1, 2) else f"bad section coding {coding}")
        if k != kind or lv != level or res != 0:
            raise ValueError(f"unexpected section header (kind {k}, level {lv}, reserved {res}) where {name} was expected")
        body = pos_b + 8
        if ln > n - body:
            raise ValueError(f"section of {name} runs past the end of the file")
        pos_b = body + ln
        return buf[body:body + ln], ln

    for l, L in enumerate(levels):
        lv = f"level {l}: "
        body, ln = section(1, l)
        r = _Reader(body)
        r.marker(sync_value(SYNC_LEVEL, l), f"before level {l} body")
        if L.mode == 3:
            nb = (L.W // 8) * (L.H // 8)
            drb = dc_raw_bits(L.dc_step)
            sym = np.zeros((nb, L.C, 64), np.int16)
            code = np.zeros((nb, L.C), np.uint8)
            for c in range(L.C):
                r.marker(sync_value(SYNC_CHANNEL, l, c), f"before level {l} channel {c}")
                code[:, c] = r.get(4, nb, lv + "token stream")
                for b in range(nb):
                    sym[b, c, 0] = r.get1(drb, lv + "token stream")
                    p = 1
                    while p < 64:
                        run = r.get1(7, lv + "token stream")
                        if run == DCT_EOB:
                            break
                        if run > 62:
                            raise ValueError(lv + f"bad run symbol {run} at block {b} (0..62 or the EOB 64)")
                        p += run
                        if p >= 64:
                            raise ValueError(lv + f"token stream runs past the 63 AC positions at block {b}")
                        mag = r.get1(8, lv + "token stream") + 1
                        sign = r.get1(1, lv + "token stream")
                        sym[b, c, zz[p]] = -mag if sign else mag
                        p += 1
            L.sym, L.code = sym.reshape(-1), code.reshape(-1)
        else:
            idx = np.empty(L.W * L.H * L.C, np.int64)
            for c in range(L.C):
                idx[c::L.C] = r.get(L.bits[c], L.W * L.H, lv + "grid indices")
            L.idx = idx
        r.marker(sync_value(SYNC_END, l), f"after level {l} body")
        if r.aligned_bytes() != ln:
            raise ValueError(lv + f"section length {ln} != the {r.aligned_bytes()} bytes its content occupies")
    lay_np = Layout(img_w, img_h, [(L.W, L.H, L.C, L.nearest) for L in levels], hidden, T=T, pos=_pos_kinds(pos))
    P = lay_np.nparams
    body, ln = section(2, 0)
    if ln != (P * 16 + 2 * SYNC_BITS + 7) // 8:
        raise ValueError(f"mlp section length {ln} != the bytes of {P} fp16 weights and two sync markers")
    r = _Reader(body)
    r.marker(sync_value(SYNC_MLP, nlevels), "before the mlp body")
    hbits = r.get(16, P, "mlp section").astype(np.uint16)
    if ((hbits & 0x7C00) == 0x7C00).any():
        raise ValueError(f"non-finite mlp weight {int(np.nonzero((hbits & 0x7C00) == 0x7C00)[0][0])}")
    p = hbits.view(np.float16).astype(np.float32)
    r.marker(sync_value(SYNC_END, nlevels), "after the mlp body")
    if pos_b != n:
        raise ValueError(f"trailing bytes after the mlp section ({n - pos_b})")
    return Ntcb(img_w, img_h, src_w, src_h, levels, hidden, p, T=T, leak=float(np.float32(leak)), clamp=clamp == 1, pos=pos,
                latent_cell=latent_cell, version=version)


def read(path: str) -> Ntcb:
    with open(path, "rb") as f:
        return parse(f.read())


def from_model_file(m: ModelFile, qbits: int = 8, latent_cell: int = 0, pos: str | None = None) -> Ntcb:
    """the container ntcb_write (main.cpp:2637-2755) writes for the state a model file holds, as saved
    at the end of a --write-ntcb run (weights already fp16 values): a DCT level 0 as its symbols and
    codes, a --qat level 0 on its palette, --qes levels on their grids (the file holds their snapped
    values), every other level at `qbits` on the per-channel min / max grid of its values"""
    lay = m.layout
    if m.size[0] < 1:
        raise ValueError("the model file carries no image size (v9 / v10)")
    if latent_cell > 255:
        raise ValueError(f"--block {latent_cell} does not fit the container's 8-bit latent_cell field")
    levels = []
    for l, ((W, H, C, nearest), off) in enumerate(zip(lay.levels, lay.offsets)):
        z = np.asarray(m.z[off:off + W * H * C], np.float32)
        if l == 0 and m.dct:
            L = NtcbLevel(W, H, C, nearest, 3, [0] * C, dc_step=m.dct["dc_step"], deadzone=1 if m.dct["deadzone"] else 0,
                          q=list(m.dct["q"]), sym=np.asarray(m.dct["sym"], np.int16).copy(), code=np.asarray(m.dct["code"], np.uint8).copy())
        elif l == 0 and m.qat > 0:
            bits = list(m.qat_ch)
            L = NtcbLevel(W, H, C, nearest, 2, bits, palette=[qat_palette(b) for b in bits], idx=np.empty(W * H * C, np.int64))
            for c in range(C):
                k = qat_index(z[c::C], bits[c])
                if not np.array_equal(L.palette[c][k], z[c::C]):
                    raise ValueError(f"a level-0 value is off its --qat grid (channel {c})")
                L.idx[c::C] = k
        elif m.qes and m.qes[l][0] > 0:
            bits, lo, hi = m.qes[l]
            L = NtcbLevel(W, H, C, nearest, 1, [bits] * C, lo=np.asarray(lo, np.float32), hi=np.asarray(hi, np.float32),
                          idx=np.empty(W * H * C, np.int64))
            levels_n = (1 << bits) - 1
            for c in range(C):
                rng = max(np.float32(L.hi[c] - L.lo[c]), np.float32(1e-6))
                k = qes_index(z[c::C], L.lo[c], rng, levels_n)
                if not np.array_equal(grid_values(L.lo[c], L.hi[c], bits)[k], z[c::C]):
                    raise ValueError(f"a level {l} --qes value is not its grid point (channel {c})")
                L.idx[c::C] = k
        else:
            if not 2 <= qbits <= 12:
                raise ValueError(f"level {l} would be stored at {qbits} bits; the container takes 2..12")
            zc = z.reshape(-1, C)
            L = NtcbLevel(W, H, C, nearest, 0, [qbits] * C, lo=zc.min(0).astype(np.float32), hi=zc.max(0).astype(np.float32),
                          idx=np.empty(W * H * C, np.int64))
            levels_n = (1 << qbits) - 1
            for c in range(C):
                rng = max(np.float32(L.hi[c] - L.lo[c]), np.float32(1e-6))
                L.idx[c::C] = q8_index(zc[:, c], L.lo[c], rng, levels_n)
        levels.append(L)
    f16_bits(m.p)
    W, H, sw, sh = m.size
    return Ntcb(W, H, sw, sh, levels, list(lay.hidden), np.asarray(m.p, np.float32).copy(), T=lay.T, leak=float(np.float32(lay.leak)),
                clamp=bool(lay.clamp_out), pos=pos if pos is not None else _spec(lay.pos), latent_cell=latent_cell)
