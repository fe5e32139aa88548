"""The oracle's restatement of the progress print's statistics against the reference's own (golden vectors from
tests/golden/make_print_stats.py: bitrate_stats as a progress print runs it, main.cpp:2273-2352 and 4171;
dct_analyze, main.cpp:1080-1208; latent_stats, main.cpp:2211-2216), and the integer histograms the oracle
exposes (the layout the device path fills) against those same figures: every figure is a sum over them."""
import ctypes as C

import numpy as np
import pytest

from oracle.oracle import DCT_COUNTS_PER_CH, DCT_COUNTS_TAIL, OrDct, print_in
from tests.golden.make_print_stats import CASES
from tests.helpers import golden

FX = golden("print_stats.npz")


def case(name):
    m, qbits, qat, qes_bits, qes_live, dct_q = CASES[name]
    g = lambda k: FX[f"{name}_{k}"]
    d = None
    if dct_q:
        W0, H0, C0, _ = m.levels[0]
        steps, code, sym = g("dct_steps").copy(), g("dct_code").copy(), g("dct_sym").copy()
        d = OrDct()
        d.C, d.BW, d.BH, d.dc_step, d.deadzone, d.lo_w16 = C0, W0 // 8, H0 // 8, 4, 0, 16
        d.step = steps.ctypes.data_as(C.POINTER(C.c_int))
        d.code = code.ctypes.data_as(C.POINTER(C.c_uint8))
        d.sym = sym.ctypes.data_as(C.POINTER(C.c_int16))
        d._keep = (steps, code, sym)
    pin = print_in(qbits=qbits, qat_ch=qat, qes_bits=qes_bits, qes_on=bool(qes_bits), qes_live=qes_live, qes_lo=g("qes_lo"),
                   qes_range=g("qes_range"), dct=d, dc_raw_bits=8)
    return m, pin, g("z").copy(), g("zdec").copy(), d


def dct_vec(s):
    return np.array(list(s.raw) + list(s.h0) + list(s.ctx) + [s.raw_total, s.h0_total, s.ctx_total, s.code_raw, s.code_h0,
                                                            s.code_ctx, s.header, s.nblk, s.ntok_nz, s.ntok_eob, s.nmag_over,
                                                            s.nz_mean, s.lnz_mean, s.eob_only_frac], np.float64)


@pytest.mark.parametrize("name", list(CASES))
def test_print_stats_match_reference(orc, name):
    m, pin, z, zdec, d = case(name)
    b, zq = orc.bitrate_stats(m, pin, m.nparams, z, zdec)
    assert np.array_equal(np.array([getattr(b, f) for f, _ in b._fields_]), FX[f"{name}_bitrate"])
    assert np.array_equal(zq.view(np.uint32), FX[f"{name}_zq"].view(np.uint32))
    lat = np.array([orc.latent_stats(m, l, z) for l in range(len(m.levels))], np.float32)
    assert np.array_equal(lat, FX[f"{name}_lat"])
    if d is not None:
        for ctx in (0, 1):
            got, want = dct_vec(orc.dct_analyze(d, 8, ctx)), FX[f"{name}_dct{ctx}"]
            assert np.allclose(got, want, rtol=1e-13, atol=0), (ctx, got - want)


def h0_of(hist, n):
    """-sum c log2(c / n) in the reference's order (ascending bin)"""
    s = 0.0
    for c in hist:
        if c:
            s -= float(c) * np.log2(float(c) / n)
    return s


def cl0_sum(hist, tot):
    return sum(float(c) * -np.log2(float(c) / tot) for c in hist if c and tot)


@pytest.mark.parametrize("name", list(CASES))
def test_print_counts_carry_the_figures(orc, name):
    """bitrate_stats' entropies and dct_analyze's per-class bits, recomputed from the oracle's histograms alone, equal the
    reference's figures: the histograms hold everything the figures need, in the documented layout"""
    m, pin, z, zdec, d = case(name)
    hb, lohi, hd = orc.print_counts(m, pin, z, zdec)
    ent = est = 0.0
    k = 0
    for l, (w, h, ch, _) in enumerate(m.levels):
        if l == 0 and d is not None:
            continue
        for c in range(ch):
            qat = l == 0 and pin.qat > 0
            qes = pin.qes_live and pin.qes_bits[l] > 0
            bits = pin.qat_ch[c] if qat else (pin.qes_bits[l] if (qes or (pin.qes_on and pin.qes_bits[l] > 0)) else pin.qbits)
            nb = 1 << bits
            hv = hb[k:k + nb]
            k += nb
            assert hv.sum() == w * h
            if not qat and not qes:   # the post-hoc scale is the channel's range
                v = z[m.offsets()[0][l] + c:m.offsets()[0][l] + w * h * ch:ch]
                assert lohi[(l * 64 + c) * 2] == v.min() and lohi[(l * 64 + c) * 2 + 1] == v.max()
            e = h0_of(hv, float(w * h))
            ent += e
            if l >= 1:
                hr = hb[k:k + nb]
                k += nb
                assert hr.sum() == w * h
                est += h0_of(hr, float(w * h))
            else:
                est += e
    assert k == hb.size
    dct_h0 = dct_ctx = 0.0
    if d is not None:
        nb = d.BW * d.BH
        tail = hd[d.C * DCT_COUNTS_PER_CH:]
        assert tail.size == DCT_COUNTS_TAIL
        want = FX[f"{name}_dct1"]
        h0 = np.zeros(7)
        ctx = np.zeros(7)
        for c in range(d.C):
            a = hd[c * DCT_COUNTS_PER_CH:(c + 1) * DCT_COUNTS_PER_CH]
            run, mag, cr, cm = a[:65], a[65:322], a[322:322 + 4160].reshape(64, 65), a[4482:4482 + 16448].reshape(64, 257)
            ctxr, ctxm, dcres = a[20930:20994], a[20994:21058], a[21058:25155]
            code, tri, pair, (nrun, neob, nsign) = a[25155:25171], a[25171:29267], a[29267:29523], a[29523:29526]
            assert run.sum() == nrun + neob and mag.sum() == nrun and nsign == nrun and dcres.sum() == nb and code.sum() == nb
            h0 += [cl0_sum(dcres, nb), cl0_sum(run, nrun + neob) - cl0_sum(run[64:], nrun + neob), cl0_sum(mag, nrun), nsign,
                   cl0_sum(run[64:], nrun + neob), cl0_sum(code, nb), 96.0]
            ctx += [cl0_sum(dcres, nb), sum(cl0_sum(cr[p, :64], ctxr[p]) for p in range(64)),
                    sum(cl0_sum(cm[p], ctxm[p]) for p in range(64)), nsign, sum(cl0_sum(cr[p, 64:], ctxr[p]) for p in range(64)),
                    -h0_of(pair, float(nb)) + h0_of(tri, float(nb)), 96.0]
        assert np.allclose(h0, want[7:14], rtol=1e-12) and np.allclose(ctx, want[14:21], rtol=1e-12)
        assert np.isclose(tail[0] / (nb * d.C), want[-3], rtol=1e-15)               # nz mean
        assert np.isclose(tail[1] / max(tail[2], 1), want[-2], rtol=1e-15)          # lnz mean
        assert np.isclose(tail[3] / (nb * d.C), want[-1], rtol=1e-15)               # eob-only fraction
        dct_h0, dct_ctx = h0.sum() - 96.0 * d.C, ctx.sum()
    want_b = FX[f"{name}_bitrate"]
    npix = m.W * m.H
    header = want_b[8]
    assert np.isclose((ent + dct_h0 + header + 16.0 * m.nparams) / npix, want_b[2], rtol=1e-12)
    assert np.isclose((est + dct_h0 + header + 16.0 * m.nparams) / npix, want_b[5], rtol=1e-12)
