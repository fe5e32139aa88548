"""Writes tests/golden/print_stats.npz: the reference's own progress-print statistics - bitrate_stats as a
progress print runs it (main.cpp:4171, order-0 in place of the context estimate), dct_analyze with and
without the code grid's context estimate, and latent_stats - for seeded latents of six layouts: continuous
levels at --qbits 8 and 6, a --qat level 0, a live --qes level, a --qes level before its start, and DCT-coded
level-0 planes with one and two channels.

Needs the reference build oracle/_ref/libntc_ref.so (oracle/Makefile, target `ref`). From the repository root:

    make -C oracle ref && python tests/golden/make_print_stats.py

Data only: the inputs (latent, decode buffer, DCT symbols / codes / steps, --qes scales) and the outputs.
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle.oracle import Model, OrDct, OrLevel, print_in, reference  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

# name: (layout, --qbits, --qat bits per level-0 channel, --qes bits per level, qes live, DCT qualities per channel)
CASES = {
    "cont2": (Model(32, 24, [(16, 12, 4, 0), (8, 6, 2, 0)], [8], T=1), 8, None, None, False, None),
    "cont2_q6": (Model(30, 22, [(15, 11, 3, 0), (7, 5, 2, 0)], [8], T=1), 6, None, None, False, None),
    "qat": (Model(24, 20, [(24, 20, 2, 1), (6, 5, 4, 0)], [8], T=4, weights=[1.0, 2.0, 0.5, 1.5]), 8, [2, 1], None, False, None),
    "qes_live": (Model(32, 24, [(16, 12, 4, 0), (8, 6, 3, 0)], [8], T=1), 8, None, [0, 5], True, None),
    "qes_pending": (Model(32, 24, [(16, 12, 4, 0), (8, 6, 3, 0)], [8], T=1), 8, None, [6, 0], False, None),
    "dct1": (Model(32, 24, [(32, 24, 1, 1), (8, 6, 4, 0)], [8], T=1), 8, None, None, False, [50]),
    "dct2": (Model(64, 48, [(64, 48, 2, 1), (16, 12, 4, 0)], [8], T=1), 8, None, [0, 8], True, [75, 30]),
    # AC symbols beyond the token magnitude cap of 256 (dct_analyze's nmag_over, main.cpp:1113, 1147)
    "dct_big": (Model(32, 24, [(32, 24, 1, 1), (8, 6, 4, 0)], [8], T=1), 8, None, None, False, [90]),
}


def case_inputs(ref, name, seed):
    """the latent, decode buffer and state of one case (the --qes scales fitted and the DCT plane snapped by the reference)"""
    m, qbits, qat, qes_bits, qes_live, dct_q = CASES[name]
    rng = np.random.default_rng(seed)
    z = rng.normal(0, 0.45, m.nz).astype(np.float32)
    if name == "cont2_q6":                      # one constant channel: the 1e-6 range floor
        z[2:m.levels[0][0] * m.levels[0][1] * 3:3] = np.float32(0.25)
    off, _ = m.offsets()
    arrs = {"z": z}
    if qat:
        grid = np.zeros((9, 257), np.float32)
        ref.lib.ref_qat_grid(grid.ctypes.data)
        n0 = m.levels[0][0] * m.levels[0][1] * m.levels[0][2]
        lv0 = z[:n0].reshape(-1, m.levels[0][2])
        for c, b in enumerate(qat):
            lv0[:, c] = grid[b][rng.integers(0, 1 << b, lv0.shape[0])]
        z[:n0] = lv0.ravel()
    zdec = z.copy()
    qlo, qrange = np.zeros(3 * 64, np.float32), np.ones(3 * 64, np.float32)
    if qes_live:
        for l, b in enumerate(qes_bits):
            if not b:
                continue
            w, h, c, nr = m.levels[l]
            L = OrLevel(w, h, c, nr, 0)
            lo, hi, rg = (np.zeros(c, np.float32) for _ in range(3))
            grid = np.zeros(c << b, np.float32)
            ref._qes_fit(C.byref(L), z[off[l]:].ctypes.data, b, lo.ctypes.data, hi.ctypes.data, rg.ctypes.data, grid.ctypes.data)
            zl, zq = z[off[l]:off[l] + w * h * c].copy(), np.zeros(w * h * c, np.float32)
            ref._qes_snap_level(C.byref(L), b, lo.ctypes.data, hi.ctypes.data, rg.ctypes.data, grid.ctypes.data, zl.ctypes.data,
                                zq.ctypes.data, 1)
            z[off[l]:off[l] + w * h * c], zdec[off[l]:off[l] + w * h * c] = zl, zq
            qlo[l * 64:l * 64 + c], qrange[l * 64:l * 64 + c] = lo, rg
    arrs.update(qes_lo=qlo, qes_range=qrange)
    d = None
    if dct_q:
        W0, H0, C0, _ = m.levels[0]
        nb = (W0 // 8) * (H0 // 8)
        steps = np.zeros(C0 * 1024, np.int32)
        for c in range(C0):
            ref._dct_build_steps(dct_q[c], 4, steps[c * 1024:].ctypes.data)
        code = rng.integers(0, 16, nb * C0).astype(np.uint8)
        code[:3] = 0                            # a few repeated codes: the context estimate has shared contexts
        sym = np.zeros(nb * C0 * 64, np.int16)
        d = OrDct()
        d.C, d.BW, d.BH, d.dc_step, d.deadzone, d.lo_w16 = C0, W0 // 8, H0 // 8, 4, 0, 16
        d.step = steps.ctypes.data_as(C.POINTER(C.c_int))
        d.code = code.ctypes.data_as(C.POINTER(C.c_uint8))
        d.sym = sym.ctypes.data_as(C.POINTER(C.c_int16))
        L0 = OrLevel(W0, H0, C0, 1, 0)
        n0 = W0 * H0 * C0
        zs, zq = np.clip(z[:n0], -1, 1).astype(np.float32), np.zeros(n0, np.float32)
        ref._dct_snap_level0(C.byref(d), C.byref(L0), zs.ctypes.data, zq.ctypes.data, None, None)
        z[:n0], zdec[:n0] = zs, zq
        if name == "dct_big":                   # large AC symbols (a snap of a [-1, 1] plane stays far below the cap)
            s3 = sym.reshape(nb * C0, 64)
            for i, (pos, val) in enumerate([(1, 300), (9, -257), (17, 256), (63, -1000), (8, 4000), (2, 257)]):
                s3[i % s3.shape[0], pos] = val
        arrs.update(dct_steps=steps, dct_code=code, dct_sym=sym)
        d._keep = (steps, code, sym)
    arrs["zdec"] = zdec
    pin = print_in(qbits=qbits, qat_ch=qat, qes_bits=qes_bits, qes_on=bool(qes_bits), qes_live=qes_live, qes_lo=qlo,
                   qes_range=qrange, dct=d, dc_raw_bits=8)
    return m, pin, arrs, d


def main():
    ref = reference()
    out = {}
    for k, name in enumerate(CASES):
        m, pin, arrs, d = case_inputs(ref, name, 100 + k)
        b, zq = ref.bitrate_stats(m, pin, m.nparams, arrs["z"], arrs["zdec"])
        out.update({f"{name}_{a}": v for a, v in arrs.items()})
        out[f"{name}_bitrate"] = np.array([getattr(b, f) for f, _ in b._fields_], np.float64)
        out[f"{name}_zq"] = zq
        out[f"{name}_lat"] = np.array([ref.latent_stats(m, l, arrs["z"]) for l in range(len(m.levels))], np.float32)
        if d is not None:
            for ctx in (0, 1):
                s = ref.dct_analyze(d, 8, ctx)
                out[f"{name}_dct{ctx}"] = np.array(list(s.raw) + list(s.h0) + list(s.ctx) +
                                                   [s.raw_total, s.h0_total, s.ctx_total, s.code_raw, s.code_h0, s.code_ctx,
                                                    s.header, s.nblk, s.ntok_nz, s.ntok_eob, s.nmag_over, s.nz_mean,
                                                    s.lnz_mean, s.eob_only_frac], np.float64)
        print(name, "bpp q8 %.4f ent %.4f est %.4f" % (b.bpp_q8, b.bpp_q8_ent, b.bpp_est))
    np.savez_compressed(os.path.join(OUT, "print_stats.npz"), **out)


if __name__ == "__main__":
    main()
