"""The progress line's statistics on the device (ntc_trainer_print_stats: an extension, the reference's --cuda
print path downloads the model and computes them on the host, main.cpp:4155-4212) against the oracle's
restatement, itself pinned to the reference's bitrate_stats / dct_analyze / latent_stats by golden vectors
(tests/test_oracle_print_stats.py): every integer histogram exact, the bitrate figures bit for bit (to 1e-13
with a live DCT plane, whose token bits are added per histogram bin instead of per token), the
quantized latent's error exact (the device's decode of the oracle's quantized latent), latent_stats to double
rounding, dct_analyze's per-class sums to 1e-12."""
import ctypes as C

import numpy as np
import pytest

from neural_block_textures_amd import synth
from neural_block_textures_amd.trainer import Layout
from oracle.oracle import OrDct, print_in
from tests.gpu_common import LAYOUTS, HostDct, data, dct_tables, qes_tables, say, trainer
from tests.test_gpu_training import full_trainer, live_dct

pytestmark = pytest.mark.gpu


def oracle_in(tr, lay, qbits, qat=None, qes_bits=None, q=None, dct=None):
    """the OrPrintIn of the trainer's state (shadow and decode buffer downloaded for the oracle only)"""
    qlo, qrg = np.zeros(3 * 64, np.float32), np.ones(3 * 64, np.float32)
    live = q is not None and q.live
    if live:
        for l in range(len(lay.levels)):
            qlo[l * 64:(l + 1) * 64] = np.array(q.lo[l][:], np.float32)
            qrg[l * 64:(l + 1) * 64] = np.array(q.range[l][:], np.float32)
    return print_in(qbits=qbits, qat_ch=qat, qes_bits=qes_bits, qes_on=bool(qes_bits), qes_live=live, qes_lo=qlo, qes_range=qrg,
                    dct=dct, dc_raw_bits=8)


def device_dct(tr, H):
    """an OrDct over the device's own symbols and codes (what the progress print reads)"""
    sym, code = tr.download_dct()
    d = OrDct()
    d.C, d.BW, d.BH, d.dc_step, d.deadzone, d.lo_w16 = H.C, H.BW, H.BH, 4, H.deadzone, H.lo16
    steps = H.steps.copy()
    d.step = steps.ctypes.data_as(C.POINTER(C.c_int))
    d.code = code.ctypes.data_as(C.POINTER(C.c_uint8))
    d.sym = sym.ctypes.data_as(C.POINTER(C.c_int16))
    d._keep = (steps, code, sym)
    return d


def check(orc, tr, lay, pin, qbits, dct=None, label=""):
    z, _ = tr.download_model()
    zdec = tr.download_zq()
    st = tr.print_stats(qbits)
    hb, lohi, hd = tr.debug_print_counts()
    ob, olohi, od = orc.print_counts(lay, pin, z, zdec)
    assert np.array_equal(hb, ob), f"{label}: bitrate histograms"
    for l, lv in enumerate(lay.levels):   # the post-hoc scale of every continuous channel
        discrete = (l == 0 and (pin.qat > 0 or pin.dct_live)) or (pin.qes_live and pin.qes_bits[l] > 0)
        for c in range(0 if discrete else lv[2]):
            assert np.array_equal(lohi[(l * 64 + c) * 2:(l * 64 + c) * 2 + 2], olohi[(l * 64 + c) * 2:(l * 64 + c) * 2 + 2]), (label, l, c)
    assert np.array_equal(hd, od), f"{label}: DCT histograms"
    b, zq = orc.bitrate_stats(lay, pin, lay.nparams, z, zdec)
    for f, _ in b._fields_:   # bit for bit; a live DCT plane's token bits are added per histogram bin, not per token
        if dct is None:
            assert getattr(st, f) == getattr(b, f), (label, f, getattr(st, f), getattr(b, f))
        else:
            assert np.isclose(getattr(st, f), getattr(b, f), rtol=1e-13, atol=0), (label, f, getattr(st, f), getattr(b, f))
    tex, wt = tr.decode_error(z=zq)                       # the device decode of the oracle's quantized latent
    assert st.q_weighted_mse == wt and np.array_equal(np.array(st.q_tex_mse[:len(tex)]), tex), label
    for l in range(len(lay.levels)):
        m, sd, mx = orc.latent_stats(lay, l, z)
        assert abs(st.lat_mean[l] - m) <= 1e-6 * max(abs(m), 1e-3) and abs(st.lat_sd[l] - sd) <= 1e-6 * sd and st.lat_max[l] == mx
    if dct is not None:
        s = orc.dct_analyze(dct, 8, 1)
        assert st.dct_live == 1 and st.dct_ntok_nz == s.ntok_nz and st.dct_ntok_eob == s.ntok_eob and st.dct_nblk == s.nblk
        for k in range(7):
            assert np.isclose(st.dct_raw[k], s.raw[k], rtol=1e-15) and np.isclose(st.dct_h0[k], s.h0[k], rtol=1e-12)
            assert np.isclose(st.dct_ctx[k], s.ctx[k], rtol=1e-12)
        assert st.dct_nz_mean == s.nz_mean and st.dct_lnz_mean == s.lnz_mean and st.dct_eob_only_frac == s.eob_only_frac
        assert st.dct_nmag_over == s.nmag_over
    say(f"{label}: bpp q{qbits} {st.bpp_q8:.4f} ent {st.bpp_q8_ent:.4f} est {st.bpp_est:.4f}, quantized mse {st.q_weighted_mse:.4f}"
        + (f", dct nz {st.dct_nz_mean:.2f} bits/blk {st.dct_raw_total / st.dct_nblk:.1f}/{st.dct_h0_total / st.dct_nblk:.1f}/"
           f"{st.dct_ctx_total / st.dct_nblk:.1f}" if dct is not None else ""))
    return st


@pytest.mark.parametrize("name,qbits", [("two_level", 8), ("rgb_16x2", 6), ("runtime", 8), ("large", 8)])
def test_print_stats_continuous(orc, name, qbits):
    lay = LAYOUTS[name]
    z, p, tgt = data(lay, 31)
    tr = trainer(lay, z, p, tgt)
    tr.lat_step(1, 0.05, 0.02, 2)
    check(orc, tr, lay, oracle_in(tr, lay, qbits), qbits, label=name)


@pytest.mark.parametrize("name,bits", [("material", [2, 3]), ("chief1_36", [2])])
def test_print_stats_qat(orc, name, bits):
    lay = LAYOUTS[name]
    grid = synth.qat_grid()
    z, p, tgt = data(lay, 32)
    n0 = lay.levels[0][0] * lay.levels[0][1] * lay.levels[0][2]
    lv0 = z[:n0].reshape(-1, lay.levels[0][2])
    for c, b in enumerate(bits):
        lv0[:, c] = synth.qat_snap(lv0[:, c], b, grid)
    z[:n0] = lv0.ravel()
    tr = trainer(lay, z, p, tgt, qat_bits=bits, qat_grid=grid)
    tr.qat_search()
    check(orc, tr, lay, oracle_in(tr, lay, 8, qat=bits), 8, label=name)


@pytest.mark.parametrize("name,bits,live", [("two_level", [0, 5], True), ("two_level", [6, 0], False), ("runtime", [0, 3, 12], True)])
def test_print_stats_qes(orc, name, bits, live):
    lay = LAYOUTS[name]
    z, p, tgt = data(lay, 33)
    tr = trainer(lay, z, p, tgt, qes_bits=bits)
    q = None
    if live:
        q, grid = qes_tables(orc, lay, z, bits)
        tr.set_qes(q, grid)
        tr.lat_step(1, 0.05, 0.02, 2)
    check(orc, tr, lay, oracle_in(tr, lay, 8, qes_bits=bits, q=q), 8, label=f"{name} qes {bits} live {live}")


@pytest.mark.parametrize("C0,q", [(1, [50]), (2, [75, 30])])
def test_print_stats_dct(orc, C0, q):
    lay = Layout(64, 48, [(64, 48, C0, True), (16, 12, 4, False)], [32, 32] if C0 == 1 else [20, 12], leak=0.01)
    z, p, tgt = data(lay, 34 + C0, zscale=0.7)
    basis, zz = dct_tables(orc)
    tr = trainer(lay, z, p, tgt, dct={"C": C0, "dc_step": 4, "q": q}, dct_basis=basis, dct_zigzag=zz)
    H = HostDct(orc, lay, q, lam=0.3)
    zd, _ = tr.download_model()
    H.probe(lay, p, tr.download_zq())
    H.snap(zd)
    tr.set_dct(H.desc(), H.code, H.sym, H.steps)
    tr.lat_step(1, 0.05, 0.02, 2)
    d = device_dct(tr, H)
    check(orc, tr, lay, oracle_in(tr, lay, 8, dct=d), 8, dct=d, label=f"dct C{C0}")


def test_print_stats_dct_large_symbols(orc):
    """AC symbols beyond the token magnitude cap (|q| > 256: a plane handed over by set_dct, as a loaded container can
    carry): the capped magnitude histogram and nmag_over, which the reference counts in both of dct_analyze's passes"""
    lay = Layout(64, 48, [(64, 48, 1, True), (16, 12, 4, False)], [32, 32], leak=0.01)
    z, p, tgt = data(lay, 36, zscale=0.7)
    basis, zz = dct_tables(orc)
    tr = trainer(lay, z, p, tgt, dct={"C": 1, "dc_step": 4, "q": [90]}, dct_basis=basis, dct_zigzag=zz)
    H = HostDct(orc, lay, [90], lam=0.3)
    zd, _ = tr.download_model()
    H.probe(lay, p, tr.download_zq())
    H.snap(zd)
    s3 = H.sym.reshape(-1, 64)
    for i, (pos, val) in enumerate([(1, 300), (9, -257), (17, 256), (63, -1000), (8, 4000), (2, 257), (3, -300)]):
        s3[7 * i, pos] = val
    tr.set_dct(H.desc(), H.code, H.sym, H.steps)   # the device rebuilds its plane from these symbols
    d = device_dct(tr, H)
    st = check(orc, tr, lay, oracle_in(tr, lay, 8, dct=d), 8, dct=d, label="dct large symbols")
    assert st.dct_nmag_over == 2 * 6


@pytest.mark.parametrize("name", ["material512", "dct512", "rgb512_two_level"])
def test_print_stats_full_size(orc, name):
    """the benchmark workloads at their full sizes after a few iterations"""
    w, lay, tr, z, p, tgt = full_trainer(name)
    d = None
    if w.dct_q:
        H = live_dct(orc, w, lay, tr, z, p, tgt)
        d = device_dct(tr, H)
    for it in range(1, 4):
        tr.mlp_step(it, w.mlp_sigma, w.mlp_lr, w.mlp_pairs, w.mlp_batch)
        tr.lat_step(it, w.lat_sigma, w.lat_lr, w.lat_pairs)
        if w.qat_bits:
            tr.qat_search()
    if d is not None:
        d = device_dct(tr, H)
    check(orc, tr, lay, oracle_in(tr, lay, 8, qat=w.qat_bits, dct=d), 8, dct=d, label=name)
