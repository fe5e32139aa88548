"""The print path's error figures on the device (an extension: the reference downloads the model and
decodes on the host to print them): mse_of (main.cpp:1764-1788) of the device's decode against the
oracle's or_mse_of (pinned to the reference's mse_of by a golden vector) on the device's decoded image
and the target. 8-bit rounding and integer sums: exact."""
import ctypes as C

import numpy as np
import pytest

from tests.gpu_common import LAYOUTS, data, say, trainer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,extent", [("material", (0, 0)), ("rgb_16x2", (50, 37)), ("large", (0, 0))])
def test_decode_error(orc, name, extent):
    lay = LAYOUTS[name]
    say("decode error", name, extent)
    z, p, tgt = data(lay, 21)
    tr = trainer(lay, z, p, tgt)
    tr.lat_step(1, 0.05, 0.02, 2)
    tex, wt = tr.decode_error(*extent)
    img = tr.decode_full()
    cw, wsum = lay.loss_weights()
    T = lay.nout // 3
    w = np.array([cw[3 * t] for t in range(T)], np.float32)
    tex_o, wt_o = np.zeros(T), C.c_double()
    orc._mse_of(img.ctypes.data, tgt.ctypes.data, lay.W, lay.H, lay.nout, w.ctypes.data, wsum, extent[0], extent[1],
                tex_o.ctypes.data, C.byref(wt_o))
    assert np.array_equal(tex, tex_o) and wt == wt_o.value, (tex, tex_o, wt, wt_o.value)


@pytest.mark.parametrize("name", ["material", "rgb_16x2"])
def test_decode_error_of_a_host_latent(orc, name):
    """the print path's second figure: the post-hoc quantized latent (here: the latent moved by a
    random amount) decoded and scored on the device, as decode_full(z) + mse_of"""
    lay = LAYOUTS[name]
    say("decode error of a host latent", name)
    z, p, tgt = data(lay, 23)
    tr = trainer(lay, z, p, tgt)
    zq = (z + np.random.default_rng(4).normal(0, 0.05, z.size)).astype(np.float32)
    tex, wt = tr.decode_error(z=zq)
    img = tr.decode_full(zq)
    cw, wsum = lay.loss_weights()
    T = lay.nout // 3
    w = np.array([cw[3 * t] for t in range(T)], np.float32)
    tex_o, wt_o = np.zeros(T), C.c_double()
    orc._mse_of(img.ctypes.data, tgt.ctypes.data, lay.W, lay.H, lay.nout, w.ctypes.data, wsum, 0, 0, tex_o.ctypes.data,
                C.byref(wt_o))
    assert np.array_equal(tex, tex_o) and wt == wt_o.value
    # and the decode buffer itself is untouched: the next figure is the model's again
    tex2, _ = tr.decode_error()
    img2 = tr.decode_full()
    orc._mse_of(img2.ctypes.data, tgt.ctypes.data, lay.W, lay.H, lay.nout, w.ctypes.data, wsum, 0, 0, tex_o.ctypes.data,
                C.byref(wt_o))
    assert np.array_equal(tex2, tex_o)
