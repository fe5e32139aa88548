"""--qes and --dct-q on the device against the oracle, exact (the reference's --cuda-check items 6
and 7, main.cpp:3152-3216): the snapped copy, the symbols, the plane, the scale codes, the proxy
bits, the truncation counts, the rate-pass bit differences and hit count."""

import numpy as np
import pytest

from neural_block_textures_amd.trainer import Layout
from tests.gpu_common import LAYOUTS, HostDct, data, dct_tables, host_snap, qes_tables, say, trainer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,bits", [("two_level", [0, 5]), ("rgb_24x2", [6]), ("runtime", [0, 3, 12]), ("jit_widths", [0, 3, 12])])
def test_qes_snap(orc, name, bits):
    lay = LAYOUTS[name]
    say("qes", name, bits)
    z, p, tgt = data(lay, 11)
    tr = trainer(lay, z, p, tgt, qes_bits=bits)
    assert np.array_equal(tr.download_zq(), z)          # not live yet: the copy is the shadow
    q, grid = qes_tables(orc, lay, z, bits)
    tr.set_qes(q, grid)
    zs, zq = host_snap(orc, lay, q, grid, z)
    assert np.array_equal(tr.download_zq(), zq)
    tr.lat_step(1, 0.05, 0.05, 2)                       # Adam moves the shadow, then the frozen snap
    zd, _ = tr.download_model()
    zs2, zq2 = host_snap(orc, lay, q, grid, zd)
    assert np.array_equal(zd, zs2)                      # the device already clamped the shadow
    assert np.array_equal(tr.download_zq(), zq2)
    assert (zq2 != zq).any()


@pytest.mark.parametrize("C0,q,deadzone,lam,rate", [(1, [50], 0, 0.0, "both"), (1, [50], 0, 0.5, "both"),
                                                    (2, [75, 30], 1, 0.3, "es"), (3, [90, 50, 20], 0, 0.4, "trunc")])
def test_dct_plane(orc, C0, q, deadzone, lam, rate):
    lay = Layout(64, 48, [(64, 48, C0, True), (16, 12, 4, False)], [32, 32] if C0 == 1 else [20, 12], leak=0.01)
    say("dct", C0, q, deadzone, lam, rate)
    z, p, tgt = data(lay, 12 + C0, zscale=0.7)
    basis, zz = dct_tables(orc)
    tr = trainer(lay, z, p, tgt, dct={"C": C0, "dc_step": 4, "q": q}, dct_basis=basis, dct_zigzag=zz)
    n0 = 64 * 48 * C0
    zc = np.clip(z[:n0], -1, 1)
    zd, _ = tr.download_model()
    assert np.array_equal(zd[:n0], zc) and np.array_equal(tr.download_zq()[:n0], zc)   # the pre-start clamp
    H = HostDct(orc, lay, q, deadzone=deadzone, lam=lam, rate=rate)
    H.probe(lay, p, np.concatenate([zc, z[n0:]]))
    zs, zq, bits, cnt = H.snap(zd)
    tr.set_dct(H.desc(), H.code, H.sym, H.steps)
    assert np.array_equal(tr.download_zq()[:n0], zq)                  # k_dct_recon on the host's symbols
    sym_d, code_d = tr.download_dct()
    assert np.array_equal(sym_d, H.sym) and np.array_equal(code_d, H.code)
    # a latent step with lr 0: the rate pass of every pair, then the snap of the unchanged shadow
    K = 3
    tr.lat_step(1, 0.05, 0.0, K)
    zd2, _ = tr.download_model()
    assert np.array_equal(zd2, zd)
    bits_d, dbits_d, nt_d, nz_d, hits_d, evals_d = tr.download_dct_rate()
    zdec = tr.download_zq()
    g_o, _, dbits_o, hits_o = orc.lat_grad(lay, p, zdec, zd2, tgt, 5, 0, 0.05, K, 3,
                                           dct=H.d if H.rate_es else None, rate_scale=float(H.rate_scale))
    if H.rate_es:
        assert np.array_equal(dbits_d, dbits_o) and hits_d == hits_o and evals_d == H.n * K
        say("dct rate hits", hits_d, "of", H.n * K)
    else:
        assert evals_d == 0
    g = tr.debug_last_zgrad()
    assert np.abs(g - g_o).max() < 1e-3 * np.sqrt((g_o.astype(np.float64) ** 2).mean())
    zs2, zq2, bits2, cnt2 = H.snap(zd2)
    sym_d, _ = tr.download_dct()
    assert np.array_equal(sym_d, H.sym) and np.array_equal(tr.download_zq()[:n0], zq2)
    if lam > 0:
        assert np.array_equal(bits_d, bits2) and nt_d == cnt2[0] and nz_d == cnt2[1]
    # a step with lr > 0 moves the shadow; the device snap of it matches the host's
    tr.lat_step(2, 0.05, 0.02, K)
    zd3, _ = tr.download_model()
    zs3, zq3, bits3, cnt3 = H.snap(zd3)
    assert np.array_equal(zd3[:n0], zs3)
    sym_d, _ = tr.download_dct()
    assert np.array_equal(sym_d, H.sym) and np.array_equal(tr.download_zq()[:n0], zq3)
    if lam > 0:
        b3, _, nt3, nz3, _, _ = tr.download_dct_rate()
        assert np.array_equal(b3, bits3) and (nt3, nz3) == (cnt3[0], cnt3[1])
    # refit: new codes from the host through set_dct, then the shadow pull (main.cpp:4110-4136)
    H.probe(lay, p, tr.download_zq())
    zs4, zq4, _, _ = H.snap(zd3)
    tr.set_dct(H.desc(), H.code, H.sym, H.steps)
    assert np.array_equal(tr.download_zq()[:n0], zq4)
    tr.shadow_pull(0, n0, 0.01)
    zp = zd3[:n0].copy()
    orc._shadow_pull(zp.ctypes.data, zq4.ctypes.data, n0, 0.01)
    zs5, zq5, _, _ = H.snap(np.concatenate([zp, zd3[n0:]]))
    zd5, _ = tr.download_model()
    assert np.array_equal(zd5[:n0], zs5) and np.array_equal(tr.download_zq()[:n0], zq5)
    # the whole plane pulls inside the re-snap's launch; a part of it through the pull kernel and then the re-snap
    tr.shadow_pull(0, n0 // 2, 0.02)
    zp = zs5.copy()
    orc._shadow_pull(zp.ctypes.data, zq5.ctypes.data, n0 // 2, 0.02)
    zs6, zq6, _, _ = H.snap(np.concatenate([zp, zd5[n0:]]))
    zd6, _ = tr.download_model()
    assert np.array_equal(zd6[:n0], zs6) and np.array_equal(tr.download_zq()[:n0], zq6)


@pytest.mark.parametrize("C0,q", [(1, [50]), (2, [75, 30])])
def test_dct_device_probe_and_refit(orc, C0, q):
    """The decoder sensitivity probe on the device (an extension: the reference probes on the host)
    against the oracle's dct_probe_codes on the same decode buffer and weights: codes equal except on a
    code boundary (the reference calls the probe an estimate); the device refit re-snaps exactly like
    the host snap with the device's codes."""
    lay = Layout(64, 48, [(64, 48, C0, True), (16, 12, 4, False)], [32, 32] if C0 == 1 else [20, 12], leak=0.01)
    say("dct probe", C0, q)
    z, p, tgt = data(lay, 40 + C0, zscale=0.7)
    basis, zz = dct_tables(orc)
    tr = trainer(lay, z, p, tgt, dct={"C": C0, "dc_step": 4, "q": q}, dct_basis=basis, dct_zigzag=zz)
    n0 = 64 * 48 * C0
    H = HostDct(orc, lay, q, lam=0.3)
    zd, _ = tr.download_model()
    H.probe(lay, p, tr.download_zq())
    H.snap(zd)
    tr.set_dct(H.desc(), H.code, H.sym, H.steps)
    tr.lat_step(1, 0.05, 0.02, 2)                        # move the shadow and the plane
    zd, pd = tr.download_model()
    code_d, gain_d = tr.dct_probe()
    H.probe(lay, pd, tr.download_zq())
    diff = np.nonzero(code_d != H.code)[0]
    say("probe codes differing", diff.size, "of", H.n)
    x = np.log2(np.maximum(gain_d.astype(np.float64), 14 / 64) / (14 / 64)) / 0.6
    assert diff.size <= max(2, H.n // 100)
    assert np.all(np.abs(code_d[diff].astype(int) - H.code[diff].astype(int)) == 1)
    assert np.all(np.abs(x[diff] - np.floor(x[diff]) - 0.5) < 1e-4)   # each one sits on a code boundary
    assert np.array_equal(np.clip(np.round(x), 0, 15).astype(np.uint8)[x < 15.5], code_d[x < 15.5])
    code_r = tr.dct_refit()
    assert np.array_equal(code_r, code_d)                 # same decoder: same probe
    H.code[:] = code_r
    zs, zq, _, _ = H.snap(zd)
    sym_d, code_dl = tr.download_dct()
    assert np.array_equal(code_dl, code_r) and np.array_equal(sym_d, H.sym)
    assert np.array_equal(tr.download_zq()[:n0], zq)
