"""Writes the golden vectors under tests/golden/ by running the reference's own CPU code.

Needs the reference build oracle/_ref/libntc_ref.so (oracle/Makefile, target `ref`: main.cpp of
the reference compiled in place with GCC's default floating point). Run from the repository root:

    make -C oracle ref && python tests/golden/make_golden.py

Every fixture is data only: seeded inputs and the reference's outputs for them.
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle.oracle import Model, OrDct, OrLevel, reference  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

# small decoder layouts covering every code path: bilinear / nearest levels, one to three levels,
# uv and lv1local positional features, 1..4 textures, image / latent ratios that are not powers of 2
LAYOUTS = {
    "b1": Model(32, 32, [(8, 8, 4, 0)], [16, 16], T=1, pos=[0], leak=0.0),
    "b2": Model(48, 40, [(12, 10, 8, 0), (5, 4, 4, 0)], [24, 20], T=1, pos=[0], leak=0.01),
    "n2": Model(40, 36, [(40, 36, 2, 1), (9, 7, 4, 0)], [32, 32], T=4, pos=[0, 1], leak=0.01, weights=[1.0, 2.0, 0.5, 1.5]),
    "n3": Model(30, 26, [(15, 13, 3, 1), (6, 5, 4, 0), (3, 3, 2, 1)], [20], T=2, pos=[1, 0], leak=0.02, clamp_out=True),
}


def P(a):
    return a.ctypes.data


def data(m: Model, seed: int):
    rng = np.random.default_rng(seed)
    z = rng.normal(0, 0.4, m.nz).astype(np.float32)
    p = rng.normal(0, 0.35, m.nparams).astype(np.float32)
    tgt = (rng.integers(0, 256, m.W * m.H * m.nout).astype(np.float32) / np.float32(255.0)).astype(np.float32)
    return z, p, tgt


def layout_arrays(m: Model):
    lv = np.array([[w, h, c, nr] for (w, h, c, nr) in m.levels], np.int32)
    return dict(W=m.W, H=m.H, T=m.T, levels=lv, hidden=np.array(m.hidden, np.int32), pos=np.array(m.pos, np.int32),
                leak=np.float32(m.leak), clamp_out=int(m.clamp_out),
                weights=np.array(m.weights or [1.0] * m.T, np.float32))


def main():
    r = reference()
    L = r.lib
    # ---- noise
    rng = np.random.default_rng(1)
    n = 4000
    keys = np.stack([rng.integers(0, 2**32, n, dtype=np.uint64), rng.integers(1, 5, n).astype(np.uint64),
                     rng.integers(0, 2**20, n).astype(np.uint64), rng.integers(0, 2**16, n).astype(np.uint64),
                     rng.integers(0, 2**40, n, dtype=np.uint64)], 1)
    keys[:8, 4] = [0, 1, 2, 3, 2**32 - 1, 2**32, 2**40 - 1, 123456789]
    g = np.array([r.gauss(*map(int, k)) for k in keys], np.float32)
    u = np.array([L.ref_noise_u32(*map(int, k)) for k in keys], np.uint32)
    nn = rng.integers(1, 2**28, n).astype(np.uint32)
    uni = np.array([L.ref_noise_uniform(int(a), int(b)) for a, b in zip(u, nn)], np.uint32)
    np.savez_compressed(os.path.join(OUT, "noise.npz"), keys=keys, gauss=g, u32=u, n=nn, uniform=uni)

    for name, m in LAYOUTS.items():
        mc = m.to_c()
        z, p, tgt = data(m, 100 + len(name))
        base = layout_arrays(m)
        # ---- decode path
        img = r.decode_full(m, p, z)
        err = r.decode_err(m, p, z, tgt)
        idx = np.random.default_rng(5).integers(0, m.W * m.H, 333).astype(np.int32)
        loss = r.loss_subset(m, p, z, tgt, idx)
        feats = np.stack([r.features(m, z, px, py) for (px, py) in [(0, 0), (m.W - 1, m.H - 1), (m.W // 3, m.H // 2), (7, 3)]])
        # ---- MLP ES step (with a second step so Adam's t = 2 path is covered)
        Pn = m.nparams
        seed, N, M, sigma, lr = 9, 6, 257, 0.02, 0.005
        pe = p.copy(); am = np.zeros(Pn, np.float32); av = np.zeros(Pn, np.float32); at = C.c_int(0)
        g1 = np.zeros(Pn, np.float32); ds = C.c_double()
        l1 = L.ref_mlp_step(C.byref(mc), P(pe), P(z), P(tgt), seed, 3, C.c_float(sigma), C.c_float(lr), N, M, P(am), P(av),
                            C.byref(at), P(g1), C.byref(ds))
        g2 = np.zeros(Pn, np.float32)
        l2 = L.ref_mlp_step(C.byref(mc), P(pe), P(z), P(tgt), seed, 4, C.c_float(sigma), C.c_float(lr), N, M, P(am), P(av),
                            C.byref(at), P(g2), C.byref(ds))
        batch = np.zeros(M, np.int32)
        L.ref_draw_batch(seed, 3, M, C.byref(mc), P(batch))
        # ---- FD step
        pf = p.copy(); fm = np.zeros(Pn, np.float32); fv = np.zeros(Pn, np.float32); ft = C.c_int(0)
        gf = np.zeros(Pn, np.float32); fr = C.c_double()
        l0 = L.ref_mlp_step_fd(C.byref(mc), P(pf), P(z), P(tgt), seed, 5, C.c_float(1e-3), C.c_float(lr), M, P(fm), P(fv),
                               C.byref(ft), P(gf), C.byref(fr))
        out = dict(base, z=z, p=p, tgt=tgt, img=img, err=err, idx=idx, loss=np.float64(loss), feats=feats,
                   es_seed=seed, es_N=N, es_M=M, es_sigma=np.float32(sigma), es_lr=np.float32(lr),
                   es_batch=batch, es_grad1=g1, es_grad2=g2, es_p=pe, es_m=am, es_v=av, es_loss1=l1, es_loss2=l2,
                   fd_grad=gf, fd_p=pf, fd_l0=l0)
        # ---- latent step (all levels, and level 0 frozen when it is nearest: the --qat mask)
        for qat in ([0, 2] if m.levels[0][3] else [0]):
            zl = z.copy(); lm_ = np.zeros(m.nz, np.float32); lv_ = np.zeros(m.nz, np.float32); lt = C.c_int(0)
            gl = np.zeros(m.nz, np.float32)
            L.ref_lat_step(C.byref(mc), P(p), P(zl), P(tgt), seed, 7, C.c_float(0.05), C.c_float(0.02), 3, qat, P(lm_),
                           P(lv_), C.byref(lt), P(gl))
            out[f"lat{qat}_grad"] = gl
            out[f"lat{qat}_z"] = zl
        # ---- qat search on a snapped level 0
        if m.levels[0][3]:
            grid = np.zeros(9 * 257, np.float32)
            L.ref_qat_grid(P(grid))
            C0 = m.levels[0][2]
            bits = np.zeros(16, np.int32)
            bits[:C0] = [2, 3, 1][:C0]
            zs = z.copy()
            n0 = m.levels[0][0] * m.levels[0][1] * C0
            for i in range(n0):
                b = int(bits[i % C0])
                zs[i] = grid[b * 257 + L.ref_qat_index(C.c_float(zs[i]), b)]
            zq = zs.copy()
            L.ref_qat_search(C.byref(mc), P(p), P(zq), P(tgt), P(bits))
            out.update(qat_bits=bits, qat_z0=zs, qat_z1=zq, qat_grid=grid)
        np.savez_compressed(os.path.join(OUT, f"model_{name}.npz"), **out)

    # ---- --qes
    rng = np.random.default_rng(3)
    qes = {}
    for bits in (2, 5, 8, 12):
        Lv = OrLevel(13, 7, 3, 0, 0)
        zz = rng.normal(0, 0.5, 13 * 7 * 3).astype(np.float32)
        lo, hi, rg = (np.zeros(3, np.float32) for _ in range(3))
        grid = np.zeros(3 << bits, np.float32)
        L.ref_qes_fit(C.byref(Lv), P(zz), bits, P(lo), P(hi), P(rg), P(grid))
        z2 = (zz * np.float32(1.3)).astype(np.float32)
        z2[:3] = [np.float32(lo[0]), np.float32(hi[1]), np.float32(lo[2] + rg[2] * 0.5)]
        zc = z2.copy(); zq = np.zeros_like(z2)
        L.ref_qes_snap_level.restype = C.c_longlong
        ch = L.ref_qes_snap_level(C.byref(Lv), bits, P(lo), P(hi), P(rg), P(grid), P(zc), P(zq), 1)
        qes.update({f"b{bits}_z": zz, f"b{bits}_lo": lo, f"b{bits}_hi": hi, f"b{bits}_range": rg, f"b{bits}_grid": grid,
                    f"b{bits}_zin": z2, f"b{bits}_zclamp": zc, f"b{bits}_zq": zq, f"b{bits}_changed": ch})
    np.savez_compressed(os.path.join(OUT, "qes.npz"), **qes)

    # ---- --dct-q
    basis = np.zeros(64, np.float32); zz = np.zeros(64, np.int32); ak = np.zeros(16, np.float32)
    L.ref_dct_tables(P(basis), P(zz), P(ak))
    steps = {}
    for q in (1, 10, 25, 49, 50, 51, 75, 90, 95, 100):
        for dc in (1, 4, 64):
            s = np.zeros(1024, np.int32)
            L.ref_dct_build_steps(q, dc, P(s))
            steps[f"q{q}_dc{dc}"] = s
    dct = dict(basis=basis, zigzag=zz, ak=ak, **{"steps_" + k: v for k, v in steps.items()})
    rng = np.random.default_rng(4)
    for case, (C0, dz, lam, lo16) in enumerate([(1, 0, 0.0, 16), (2, 1, 0.0, 4), (3, 0, 0.6, 4), (4, 1, 0.05, 16)]):
        W = H = 24
        BW = BH = 3
        L0 = OrLevel(W, H, C0, 1, 0)
        st = np.zeros(C0 * 1024, np.int32)
        for c in range(C0):
            L.ref_dct_build_steps([50, 75, 30, 90][c], 4, P(st[c * 1024:]))
        code = rng.integers(0, 16, BW * BH * C0).astype(np.uint8)
        zin = rng.normal(0, 0.6, W * H * C0).astype(np.float32)
        lamt = np.array([np.float32(lam / (((14 / 64) * 2 ** (0.6 * k)) ** 2 * 16.0)) for k in range(16)], np.float32)
        sym = np.zeros(BW * BH * C0 * 64, np.int16)
        d = OrDct()
        d.C, d.BW, d.BH, d.dc_step, d.deadzone, d.lo_w16 = C0, BW, BH, 4, dz, lo16
        for k in range(16):
            d.lam_t16[k] = lamt[k]
        d.step = st.ctypes.data_as(C.POINTER(C.c_int)); d.code = code.ctypes.data_as(C.POINTER(C.c_uint8))
        d.sym = sym.ctypes.data_as(C.POINTER(C.c_int16))
        zs = zin.copy(); zq = np.zeros_like(zin); bits = np.zeros(BW * BH * C0, np.int32); cnt = np.zeros(3, np.int64)
        L.ref_dct_snap_level0(C.byref(d), C.byref(L0), P(zs), P(zq), P(bits), P(cnt))
        zr = np.zeros_like(zin); bits2 = np.zeros_like(bits)
        L.ref_dct_recon_level0(C.byref(d), C.byref(L0), P(zr), P(bits2))
        eps = rng.normal(0, 1, W * H * C0).astype(np.float32)
        db = np.zeros(BW * BH * C0, np.int32)
        L.ref_dct_rate_pair(C.byref(d), C.byref(L0), P(zs), P(eps), C.c_float(0.05), P(db))
        dct.update({f"c{case}_cfg": np.array([C0, dz, lo16, BW, BH, 4]), f"c{case}_lam": lamt, f"c{case}_steps": st,
                    f"c{case}_code": code, f"c{case}_zin": zin, f"c{case}_z": zs, f"c{case}_zq": zq,
                    f"c{case}_sym": sym.copy(), f"c{case}_bits": bits, f"c{case}_counts": cnt, f"c{case}_recon": zr,
                    f"c{case}_eps": eps, f"c{case}_dbits": db})
    # probe codes on a small DCT model (level 0 full-resolution nearest, 2 channels)
    m = Model(24, 16, [(24, 16, 2, 1), (6, 4, 4, 0)], [16, 16], T=1, pos=[0], leak=0.01)
    zmod, pmod, _ = data(m, 77)
    zmod[: 24 * 16 * 2] = np.clip(zmod[: 24 * 16 * 2], -1, 1)
    d = OrDct()
    d.C, d.BW, d.BH, d.dc_step, d.deadzone, d.lo_w16 = 2, 3, 2, 4, 1, 16
    code = np.zeros(12, np.uint8)
    st = np.zeros(2048, np.int32)
    d.step = st.ctypes.data_as(C.POINTER(C.c_int)); d.code = code.ctypes.data_as(C.POINTER(C.c_uint8))
    symp = np.zeros(12 * 64, np.int16); d.sym = symp.ctypes.data_as(C.POINTER(C.c_int16))
    L.ref_dct_probe_codes(C.byref(m.to_c()), P(pmod), P(zmod), C.byref(d), P(code))
    dct.update(probe_z=zmod, probe_p=pmod, probe_code=code.copy(), probe_layout=np.array([24, 16, 2, 6, 4, 4]))
    np.savez_compressed(os.path.join(OUT, "dct.npz"), **dct)

    # ---- fp16 round trip
    rng = np.random.default_rng(6)
    xs = np.concatenate([rng.normal(0, 3, 3000), rng.normal(0, 1e-5, 500), [65504, 65519.99, 1.0004883, 5.9604645e-8]]).astype(np.float32)
    ov = C.c_int()
    h = np.array([L.ref_f32_to_f16(C.c_float(x), C.byref(ov)) for x in xs], np.uint16)
    back = np.array([L.ref_f16_to_f32(int(v)) for v in range(65536)], np.float32)
    np.savez_compressed(os.path.join(OUT, "fp16.npz"), x=xs, half=h, all_back=back)
    # ---- the printed error (mse_of): two textures, values outside [0, 1] and on 8-bit rounding boundaries,
    # the whole image and a partial extent
    rng = np.random.default_rng(8)
    W, H, nc = 37, 29, 6
    a = rng.normal(0.5, 0.4, W * H * nc).astype(np.float32)
    b = rng.random(W * H * nc).astype(np.float32)
    a[:300] = (np.arange(300) % 256 + 0.5).astype(np.float32) / np.float32(255.0)   # k + 1/2 LSB: lround's half cases
    wts = np.array([1.0, 2.5], np.float32)
    mse = dict(a=a, b=b, shape=np.array([W, H, nc]), w=wts, wsum=np.float32(3.5))
    for tag, (ew, eh) in {"full": (0, 0), "part": (30, 20)}.items():
        tex, wt = np.zeros(2), C.c_double()
        L.ref_mse_of(P(a), P(b), W, H, nc, P(wts), C.c_float(3.5), ew, eh, P(tex), C.byref(wt))
        mse[f"tex_{tag}"], mse[f"weighted_{tag}"], mse[f"extent_{tag}"] = tex, np.float64(wt.value), np.array([ew, eh])
    np.savez_compressed(os.path.join(OUT, "mse.npz"), **mse)
    print("golden vectors written to", OUT)


if __name__ == "__main__":
    main()
