"""The oracle against the golden vectors the reference's own CPU code wrote (tests/golden/,
made by tests/golden/make_golden.py from main.cpp compiled in place). Every comparison is exact:
the oracle restates the reference's evaluation order, FMA placement included."""
import ctypes as C

import numpy as np
import pytest

from oracle.oracle import OrDct, OrLevel, model_of
from tests.helpers import golden, layout_of

MODELS = ["b1", "b2", "n2", "n3"]


def test_noise_keys(orc):
    fx = golden("noise.npz")
    k = fx["keys"]
    g = np.array([orc.gauss(*map(int, row)) for row in k], np.float32)
    u = np.array([orc._noise_u32(*map(int, row)) for row in k], np.uint32)
    uni = np.array([orc._noise_uniform(int(a), int(b)) for a, b in zip(fx["u32"], fx["n"])], np.uint32)
    assert np.array_equal(g.view(np.uint32), fx["gauss"].view(np.uint32))
    assert np.array_equal(u, fx["u32"])
    assert np.array_equal(uni, fx["uniform"])


@pytest.mark.parametrize("name", MODELS)
def test_decode_path(orc, name):
    fx = golden(f"model_{name}.npz")
    lay = layout_of(fx)
    z, p, tgt = fx["z"], fx["p"], fx["tgt"]
    assert np.array_equal(orc.decode_full(lay, p, z), fx["img"])
    assert np.array_equal(orc.decode_err(lay, p, z, tgt), fx["err"])
    assert orc.loss_subset(lay, p, z, tgt, fx["idx"]) == float(fx["loss"])
    pts = [(0, 0), (lay.W - 1, lay.H - 1), (lay.W // 3, lay.H // 2), (7, 3)]
    for (px, py), want in zip(pts, fx["feats"]):
        assert np.array_equal(orc.features(lay, z, px, py), want)


@pytest.mark.parametrize("name", MODELS)
def test_mlp_es_two_steps(orc, name):
    fx = golden(f"model_{name}.npz")
    lay = layout_of(fx)
    z, tgt = fx["z"], fx["tgt"]
    seed, N, M, sigma, lr = int(fx["es_seed"]), int(fx["es_N"]), int(fx["es_M"]), float(fx["es_sigma"]), float(fx["es_lr"])
    p = fx["p"].copy()
    P = p.size
    am, av = np.zeros(P, np.float32), np.zeros(P, np.float32)
    for t, it, gkey in [(1, 3, "es_grad1"), (2, 4, "es_grad2")]:
        idx = orc.draw_batch(seed, it, M, lay.W * lay.H)
        if it == 3:
            assert np.array_equal(idx, fx["es_batch"])
        dl, _, _, _ = orc.mlp_es_eval(lay, p, z, tgt, seed, it, sigma, N, idx)
        g = orc.mlp_es_grad(P, N, seed, it, sigma, dl)
        assert np.array_equal(g, fx[gkey]), f"ES gradient of step {t}"
        orc.adam(p, g, am, av, lr, t)
    assert np.array_equal(p, fx["es_p"]) and np.array_equal(am, fx["es_m"]) and np.array_equal(av, fx["es_v"])


@pytest.mark.parametrize("name", MODELS)
def test_mlp_fd_step(orc, name):
    fx = golden(f"model_{name}.npz")
    lay = layout_of(fx)
    z, tgt, p = fx["z"], fx["tgt"], fx["p"].copy()
    M, seed = int(fx["es_M"]), int(fx["es_seed"])
    idx = orc.draw_batch(seed, 5, M, lay.W * lay.H)
    dl, hh, l0 = orc.mlp_fd_eval(lay, p, z, tgt, np.float32(1e-3), idx)
    g = orc.fd_grad(dl, hh)
    assert np.array_equal(g, fx["fd_grad"])
    assert l0 == float(fx["fd_l0"])
    am, av = np.zeros(p.size, np.float32), np.zeros(p.size, np.float32)
    orc.adam(p, g, am, av, float(fx["es_lr"]), 1)
    assert np.array_equal(p, fx["fd_p"])


@pytest.mark.parametrize("name", MODELS)
def test_latent_step(orc, name):
    fx = golden(f"model_{name}.npz")
    lay = layout_of(fx)
    z, p, tgt = fx["z"], fx["p"], fx["tgt"]
    for qat in ([0, 2] if lay.levels[0][3] else [0]):
        mask = sum(1 << l for l in range(len(lay.levels)) if not (qat and l == 0))
        g, dpix, _, _ = orc.lat_grad(lay, p, z, z, tgt, int(fx["es_seed"]), 7, 0.05, 3, mask, want_dpix=True)
        assert np.array_equal(g, fx[f"lat{qat}_grad"])
        # the scatter alone, from the same per-pixel differences and the step's Gaussians (stream 1)
        eps = np.concatenate([orc.gauss_fill(int(fx["es_seed"]), 1, 7, k, 0, lay.nz) for k in range(3)])
        assert np.array_equal(orc.lat_scatter(lay, eps, dpix, 3, mask, np.float32(0.05)), fx[f"lat{qat}_grad"])
        zz = z.copy()
        orc.adam(zz, g, np.zeros_like(zz), np.zeros_like(zz), 0.02, 1)
        assert np.array_equal(zz, fx[f"lat{qat}_z"])


@pytest.mark.parametrize("name", [n for n in MODELS if golden(f"model_{n}.npz").get("qat_bits") is not None])
def test_qat_search(orc, name):
    fx = golden(f"model_{name}.npz")
    lay = layout_of(fx)
    grid = np.zeros(9 * 257, np.float32)
    orc._qat_grid(grid.ctypes.data)
    assert np.array_equal(grid, fx["qat_grid"])
    z = fx["qat_z0"].copy()
    orc.qat_search(lay, fx["p"], z, fx["tgt"], [int(b) for b in fx["qat_bits"][: lay.levels[0][2]]], grid)
    assert np.array_equal(z, fx["qat_z1"])
    assert not np.array_equal(fx["qat_z0"], fx["qat_z1"])   # the search moved something


def test_qes(orc):
    fx = golden("qes.npz")
    for bits in (2, 5, 8, 12):
        L = OrLevel(13, 7, 3, 0, 0)
        zz = fx[f"b{bits}_z"]
        lo, hi, rg = (np.zeros(3, np.float32) for _ in range(3))
        grid = np.zeros(3 << bits, np.float32)
        orc._qes_fit(C.byref(L), zz.ctypes.data, bits, lo.ctypes.data, hi.ctypes.data, rg.ctypes.data, grid.ctypes.data)
        for k in ("lo", "hi", "range", "grid"):
            assert np.array_equal(locals()[{"lo": "lo", "hi": "hi", "range": "rg", "grid": "grid"}[k]], fx[f"b{bits}_{k}"])
        zc = fx[f"b{bits}_zin"].copy()
        zq = np.zeros_like(zc)
        ch = orc._qes_snap_level(C.byref(L), bits, lo.ctypes.data, hi.ctypes.data, rg.ctypes.data, grid.ctypes.data,
                                 zc.ctypes.data, zq.ctypes.data, 1)
        assert np.array_equal(zc, fx[f"b{bits}_zclamp"]) and np.array_equal(zq, fx[f"b{bits}_zq"])
        assert ch == int(fx[f"b{bits}_changed"])


def _dct(case, fx):
    C0, dz, lo16, BW, BH, dc = (int(x) for x in fx[f"c{case}_cfg"])
    d = OrDct()
    d.C, d.BW, d.BH, d.dc_step, d.deadzone, d.lo_w16 = C0, BW, BH, dc, dz, lo16
    lam = fx[f"c{case}_lam"]
    for k in range(16):
        d.lam_t16[k] = lam[k]
    st = fx[f"c{case}_steps"].copy()
    code = fx[f"c{case}_code"].copy()
    sym = np.zeros(BW * BH * C0 * 64, np.int16)
    d.step = st.ctypes.data_as(C.POINTER(C.c_int))
    d.code = code.ctypes.data_as(C.POINTER(C.c_uint8))
    d.sym = sym.ctypes.data_as(C.POINTER(C.c_int16))
    return d, (st, code, sym), OrLevel(BW * 8, BH * 8, C0, 1, 0)


def test_dct_tables_and_steps(orc):
    fx = golden("dct.npz")
    b, z, a = np.zeros(64, np.float32), np.zeros(64, np.int32), np.zeros(16, np.float32)
    orc.lib.or_dct_tables(b.ctypes.data, z.ctypes.data, a.ctypes.data)
    assert np.array_equal(b.view(np.uint32), fx["basis"].view(np.uint32))
    assert np.array_equal(z, fx["zigzag"]) and np.array_equal(a.view(np.uint32), fx["ak"].view(np.uint32))
    for k in fx:
        if k.startswith("steps_q"):
            q, dc = (int(x[1:]) if x[0] == "q" else int(x[2:]) for x in k[6:].split("_"))
            s = np.zeros(1024, np.int32)
            orc._dct_build_steps(q, dc, s.ctypes.data)
            assert np.array_equal(s, fx[k]), k


@pytest.mark.parametrize("case", range(4))
def test_dct_snap_recon_rate(orc, case):
    fx = golden("dct.npz")
    d, keep, L0 = _dct(case, fx)
    zs = fx[f"c{case}_zin"].copy()
    zq = np.zeros_like(zs)
    bits = np.zeros(d.BW * d.BH * d.C, np.int32)
    cnt = np.zeros(3, np.int64)
    orc._dct_snap_level0(C.byref(d), C.byref(L0), zs.ctypes.data, zq.ctypes.data, bits.ctypes.data, cnt.ctypes.data)
    assert np.array_equal(zs, fx[f"c{case}_z"]) and np.array_equal(zq, fx[f"c{case}_zq"])
    assert np.array_equal(keep[2], fx[f"c{case}_sym"])
    if float(fx[f"c{case}_lam"].max()) > 0:
        assert np.array_equal(bits, fx[f"c{case}_bits"])
    assert np.array_equal(cnt, fx[f"c{case}_counts"])
    zr = np.zeros_like(zs)
    orc._dct_recon_level0(C.byref(d), C.byref(L0), zr.ctypes.data, None)
    assert np.array_equal(zr, fx[f"c{case}_recon"])
    db = np.zeros(d.BW * d.BH * d.C, np.int32)
    orc._dct_rate_pair(C.byref(d), C.byref(L0), zs.ctypes.data, fx[f"c{case}_eps"].ctypes.data, 0.05, db.ctypes.data)
    assert np.array_equal(db, fx[f"c{case}_dbits"])


def test_dct_probe_codes(orc):
    from oracle.oracle import Model
    fx = golden("dct.npz")
    m = Model(24, 16, [(24, 16, 2, 1), (6, 4, 4, 0)], [16, 16], T=1, pos=[0], leak=0.01)
    d = OrDct()
    d.C, d.BW, d.BH, d.dc_step, d.deadzone, d.lo_w16 = 2, 3, 2, 4, 1, 16
    code = np.zeros(12, np.uint8)
    orc._dct_probe_codes(C.byref(m.to_c()), fx["probe_p"].ctypes.data, fx["probe_z"].ctypes.data, C.byref(d),
                         code.ctypes.data)
    assert np.array_equal(code, fx["probe_code"])


def test_fp16(orc):
    fx = golden("fp16.npz")
    ov = C.c_int()
    h = np.array([orc._f32_to_f16(float(x), C.addressof(ov)) for x in fx["x"]], np.uint16)
    assert np.array_equal(h, fx["half"])
    back = np.array([orc._f16_to_f32(v) for v in range(65536)], np.float32)
    assert np.array_equal(back.view(np.uint32), fx["all_back"].view(np.uint32))


def test_mse_of(orc):
    """the printed error (mse_of) against the reference's, whole image and a partial extent"""
    fx = golden("mse.npz")
    W, H, nc = (int(v) for v in fx["shape"])
    a, b, w = fx["a"], fx["b"], fx["w"]
    for tag in ("full", "part"):
        ew, eh = (int(v) for v in fx[f"extent_{tag}"])
        tex, wt = np.zeros(2), C.c_double()
        orc._mse_of(a.ctypes.data, b.ctypes.data, W, H, nc, w.ctypes.data, float(fx["wsum"]), ew, eh, tex.ctypes.data, C.byref(wt))
        assert np.array_equal(tex, fx[f"tex_{tag}"]) and wt.value == float(fx[f"weighted_{tag}"])
