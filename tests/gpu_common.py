"""Layouts and helpers of the GPU parity tests (HIP path through the C ABI against the oracle)."""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

from neural_block_textures_amd import synth
from neural_block_textures_amd.trainer import PK_LV1LOCAL, PK_UV, DctDesc, Layout, QesDesc, Trainer
from oracle.oracle import OrDct, OrLevel

# One layout per compiled MLP shape, at sizes the oracle finishes in seconds, plus one that runs
# through the runtime-shaped kernels (3 levels, lv1local, clamp output, ratios not powers of 2).
LAYOUTS = {
    "rgb_16x2": Layout(64, 64, [(16, 16, 4, False)], [16, 16], leak=0.0),
    "rgb_24x2": Layout(48, 48, [(12, 12, 4, False)], [24, 24], leak=0.01),
    "two_level": Layout(96, 64, [(24, 16, 8, False), (6, 4, 4, False)], [32, 32], leak=0.0),
    "material": Layout(48, 40, [(48, 40, 2, True), (12, 10, 4, False)], [32, 32], T=4, leak=0.01,
                       weights=[1.0, 2.0, 0.5, 1.5]),
    "dct_plane": Layout(64, 48, [(64, 48, 1, True), (16, 12, 4, False)], [32, 32], leak=0.01),
    "large": Layout(48, 48, [(24, 24, 4, False), (6, 6, 8, False)], [64, 64], T=4, leak=0.0),
    "runtime": Layout(50, 38, [(13, 10, 3, True), (5, 4, 4, False), (3, 3, 2, False)], [20, 12], T=2,
                      pos=[PK_LV1LOCAL, PK_UV], leak=0.02, clamp_out=True, weights=[1.0, 3.0]),
    # the reference's published runs (README.md:358, 382, 531): selector plane, nearest block latent,
    # lv1local, hidden widths that pad the matrix tiles (36 -> 48, 27 -> 32)
    "chief1_36": Layout(64, 48, [(64, 48, 1, True), (16, 12, 2, True)], [36, 36], pos=[PK_LV1LOCAL], leak=1 / 1024),
    "mat_qat_36": Layout(48, 40, [(48, 40, 2, True), (12, 10, 4, True)], [36, 36], T=4, pos=[PK_LV1LOCAL],
                         leak=1 / 1024, weights=[1.0, 2.0, 0.5, 1.5]),
    "image3_27": Layout(64, 48, [(64, 48, 1, True), (8, 6, 4, False)], [27, 27], pos=[PK_LV1LOCAL], leak=1 / 1024),
    # README.md:620's 17-wide DCT decoder: 2 hidden tiles, the second with one unit
    "dct_17": Layout(64, 48, [(64, 48, 1, True), (16, 12, 4, False)], [17, 17], pos=[PK_LV1LOCAL], leak=1 / 1024),
    # an 11-wide decoder (7-11-11-3): one partial hidden tile, so the population kernel's pixel-per-lane output layer
    # with three k-steps of hidden inputs
    "dct_11": Layout(64, 48, [(64, 48, 1, True), (16, 12, 4, False)], [11, 11], pos=[PK_LV1LOCAL], leak=1 / 1024),
    # README.md:991's 3-texture material (9 outputs) and README.md:298's 4-texture --qat 2 with a 4-channel block
    "run8x3": Layout(64, 48, [(32, 24, 8, False), (16, 12, 4, False)], [24, 24], T=3, weights=[1.0, 1.0, 0.5]),
    "mat_qat1x4_36": Layout(48, 40, [(48, 40, 1, True), (12, 10, 4, True)], [36, 36], T=4, pos=[PK_LV1LOCAL],
                            leak=1 / 1024),
    # shapes the library does not list: kernels specialised at init (hipRTC); VALU only, and with the
    # matrix cores
    "jit_valu_7": Layout(64, 48, [(16, 12, 4, False)], [7, 7], leak=0.01),
    "jit_mfma_28": Layout(48, 40, [(48, 40, 2, True), (12, 10, 4, False)], [28, 28], T=4, pos=[PK_LV1LOCAL], leak=0.01,
                          weights=[1.0, 0.5, 2.0, 1.0]),
    # a 13-wide RGB decoder specialised at init: the pixel-per-lane output layer on a partial hidden tile
    "jit_own_13": Layout(64, 48, [(16, 12, 4, False)], [13, 13], leak=0.01),
}
# the same layouts with every stage forced onto the VALU kernels (ntc_trainer_set_matrix_cores(0))
for _name in ("material", "chief1_36"):
    _lay = Layout(**{k: getattr(LAYOUTS[_name], k) for k in LAYOUTS[_name].__dataclass_fields__})
    _lay.valu_only = True
    LAYOUTS[_name + "_valu"] = _lay
# the material layout with --clamp outputs (the matrix-core kernels' clamped instances)
LAYOUTS["material_clamp"] = Layout(**{k: getattr(LAYOUTS["material"], k) for k in LAYOUTS["material"].__dataclass_fields__})
LAYOUTS["material_clamp"].clamp_out = True
# "runtime" (hidden widths 20, 12) on the runtime-shaped kernels, and the same model on the kernels
# specialised at init for its widths (FixedShapeW)
LAYOUTS["jit_widths"] = Layout(**{k: getattr(LAYOUTS["runtime"], k) for k in LAYOUTS["runtime"].__dataclass_fields__})
LAYOUTS["runtime"].runtime_kernels = True


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def data(layout: Layout, seed: int, zscale=0.4):
    rng = np.random.default_rng(seed)
    z = rng.normal(0, zscale, layout.nz).astype(np.float32)
    p = synth.init_model(layout, seed)[1]
    p = (p + rng.normal(0, 0.05, p.size)).astype(np.float32)   # nonzero biases
    tgt = (rng.integers(0, 256, layout.W * layout.H * layout.nout).astype(np.float32) / np.float32(255.0))
    return z, p, tgt.astype(np.float32)


def trainer(layout: Layout, z, p, tgt, *, max_pairs=64, max_batch=4096, seed=5, **kw):
    tr = Trainer()
    d = Trainer.model_desc(layout, max_pairs=max_pairs, max_batch=max_batch, seed=seed, **kw)
    if getattr(layout, "runtime_kernels", False):   # NTC_HIP_JIT=0: the runtime-shaped kernels, not specialised ones
        old = os.environ.get("NTC_HIP_JIT")
        os.environ["NTC_HIP_JIT"] = "0"
        try:
            tr.init(d, z, p, tgt, layout)
        finally:
            if old is None:
                del os.environ["NTC_HIP_JIT"]
            else:
                os.environ["NTC_HIP_JIT"] = old
    else:
        tr.init(d, z, p, tgt, layout)
    if getattr(layout, "valu_only", False):
        tr.set_matrix_cores(False)
    return tr


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.abs(a - b) / np.maximum(np.abs(b), 1e-300)


def dct_tables(orc):
    b, zz, ak = np.zeros(64, np.float32), np.zeros(64, np.int32), np.zeros(16, np.float32)
    orc.lib.or_dct_tables(b.ctypes.data, zz.ctypes.data, ak.ctypes.data)
    return b, zz


class HostDct:
    """The host side of a DCT-coded level 0: codes, symbols, steps, bits (the oracle computes them)."""

    def __init__(self, orc, lay, q, dc_step=4, deadzone=0, lam=0.0, lo16=4, rate="both"):
        self.orc = orc
        W, H, C0, _ = lay.levels[0]
        self.L0 = OrLevel(W, H, C0, 1, 0)
        self.C, self.BW, self.BH = C0, W // 8, H // 8
        self.n = self.BW * self.BH * C0
        self.steps = np.zeros(C0 * 1024, np.int32)
        for c in range(C0):
            orc._dct_build_steps(q[c], dc_step, self.steps[c * 1024:].ctypes.data)
        self.code = np.zeros(self.n, np.uint8)
        self.sym = np.zeros(self.n * 64, np.int16)
        self.rate_es = lam > 0 and rate != "trunc"
        self.rate_trunc = lam > 0 and rate != "es"
        gk = lambda k: (14 / 64) * 2 ** (0.6 * k)
        self.lam_t16 = np.array([np.float32(lam / (gk(k) * gk(k) * 16.0)) if self.rate_trunc else 0.0
                                 for k in range(16)], np.float32)
        self.rate_scale = np.float32(lam / (16.0 * 65025.0 * lay.W * lay.H)) if self.rate_es else np.float32(0)
        self.d = OrDct()
        self.d.C, self.d.BW, self.d.BH, self.d.dc_step, self.d.deadzone, self.d.lo_w16 = C0, self.BW, self.BH, dc_step, deadzone, lo16
        for k in range(16):
            self.d.lam_t16[k] = self.lam_t16[k]
        self.d.step = self.steps.ctypes.data_as(C.POINTER(C.c_int))
        self.d.code = self.code.ctypes.data_as(C.POINTER(C.c_uint8))
        self.d.sym = self.sym.ctypes.data_as(C.POINTER(C.c_int16))
        self.dc_step, self.deadzone, self.lo16 = dc_step, deadzone, lo16

    def desc(self):
        d = DctDesc()
        d.live, d.C, d.BW, d.BH, d.N, d.dc_step = 1, self.C, self.BW, self.BH, 8, self.dc_step
        d.rate_es, d.rate_trunc, d.rate_scale = int(self.rate_es), int(self.rate_trunc), self.rate_scale
        for k in range(16):
            d.lam_t16[k] = self.lam_t16[k]
        d.lo_w16, d.deadzone = self.lo16, self.deadzone
        return d

    def probe(self, lay, p, zdec):
        self.orc._dct_probe_codes(C.byref(__import__("oracle.oracle", fromlist=["model_of"]).model_of(lay)),
                                  p.ctypes.data, zdec.ctypes.data, C.byref(self.d), self.code.ctypes.data)

    def snap(self, z):
        """dct_snap_level0 on a copy: (clamped shadow, plane, bits, counts); symbols land in self.sym"""
        n0 = self.L0.W * self.L0.H * self.C
        zs, zq = z[:n0].copy(), np.zeros(n0, np.float32)
        bits, cnt = np.zeros(self.n, np.int32), np.zeros(3, np.int64)
        self.orc._dct_snap_level0(C.byref(self.d), C.byref(self.L0), zs.ctypes.data, zq.ctypes.data, bits.ctypes.data,
                                  cnt.ctypes.data)
        return zs, zq, bits, cnt


def qes_tables(orc, lay, z, bits_per_level):
    q = QesDesc()
    grid_all = []
    off = 0
    for l, bits in enumerate(bits_per_level):
        w, h, c, nr = lay.levels[l]
        if bits:
            L = OrLevel(w, h, c, int(nr), 0)
            lo, hi, rg = (np.zeros(c, np.float32) for _ in range(3))
            grid = np.zeros(c << bits, np.float32)
            orc._qes_fit(C.byref(L), z[off:].ctypes.data, bits, lo.ctypes.data, hi.ctypes.data, rg.ctypes.data,
                         grid.ctypes.data)
            q.bits[l] = bits
            for ch in range(c):
                q.lo[l][ch], q.hi[l][ch], q.range[l][ch] = lo[ch], hi[ch], rg[ch]
                q.grid_off[l][ch] = sum(g.size for g in grid_all) + ch * (1 << bits)
            grid_all.append(grid)
        off += w * h * c
    q.live, q.frozen = 1, 1
    return q, np.concatenate(grid_all)


def host_snap(orc, lay, q, grid, z):
    """Decoder::qes_refresh on a copy of the shadow: (clamped shadow, snapped copy)"""
    z = z.copy()
    zq = z.copy()
    off = 0
    for l, (w, h, c, nr) in enumerate(lay.levels):
        n = w * h * c
        if q.bits[l]:
            L = OrLevel(w, h, c, int(nr), 0)
            lo = np.array(q.lo[l][:c], np.float32); hi = np.array(q.hi[l][:c], np.float32)
            rg = np.array(q.range[l][:c], np.float32)
            g = grid[q.grid_off[l][0]:q.grid_off[l][0] + (c << q.bits[l])].copy()
            zl, zql = z[off:off + n].copy(), np.zeros(n, np.float32)
            orc._qes_snap_level(C.byref(L), int(q.bits[l]), lo.ctypes.data, hi.ctypes.data, rg.ctypes.data,
                                g.ctypes.data, zl.ctypes.data, zql.ctypes.data, 1)
            z[off:off + n], zq[off:off + n] = zl, zql
        off += n
    return z, zq
