"""ntc_trainer_decode_error_noalloc (no allocation at call time; partial sums in the library's static
per-GPU scratch) against ntc_trainer_decode_error (per-call allocation) through the C ABI: identical
figures (integer sums of squared 8-bit differences, exact), on two calls in a row - the second over a
smaller extent, so the scratch still holds the first call's larger set of partials - and with a host
latent, on RGB and 4-texture models, and on two trainers of different sizes on the same GPU; the library's own
count of its hipMalloc / hipFree calls is unchanged across every no-allocation call."""
import numpy as np
import pytest

from neural_block_textures_amd import synth
from neural_block_textures_amd.trainer import Layout
from tests.gpu_common import LAYOUTS, data, say, trainer

pytestmark = pytest.mark.gpu


def same(a, b):
    (ta, wa), (tb, wb) = a, b
    return np.array_equal(ta, tb) and wa == wb


@pytest.mark.parametrize("name", ["rgb_16x2", "material", "runtime"])
def test_noalloc_matches_decode_error(orc, name):
    lay = LAYOUTS[name]
    say("noalloc", name)
    z, p, tgt = data(lay, 21)
    tr = trainer(lay, z, p, tgt)
    full = tr.decode_error()
    assert full[1] > 0
    before = tr.device_allocations()
    assert same(tr.decode_error_noalloc(), full)                                  # whole image
    assert tr.device_allocations() == before                                      # no hipMalloc / hipFree in the call
    ew, eh = lay.W - 7, lay.H // 2
    small = tr.decode_error(ew, eh)
    assert same(tr.decode_error_noalloc(ew, eh), small)                           # then a smaller extent
    assert not same(small, full)
    zq = np.round(z * 4) / 4
    want = tr.decode_error(z=zq)
    a0 = tr.device_allocations()
    got = tr.decode_error_noalloc(z=zq)                                          # a host latent
    assert tr.device_allocations() == a0 and same(got, want)
    assert same(tr.decode_error_noalloc(), full)                                  # and the decode buffer again
    assert tr.device_allocations() == a0
    tr.decode_error()
    a1 = tr.device_allocations()                                                  # the allocating entry point counts
    assert a1[0] == a0[0] + 1 and a1[1] == a0[1] + 1
    # the oracle's mse_of (pinned to the reference's by a golden vector) of the device's decode
    cw, wsum = lay.loss_weights()
    T = lay.nout // 3
    w = np.array([cw[3 * t] for t in range(T)], np.float32)
    tex_o, w_o = np.zeros(T), np.zeros(1)
    img = tr.decode_full()
    orc._mse_of(img.ctypes.data, tgt.ctypes.data, lay.W, lay.H, lay.nout, w.ctypes.data, wsum, 0, 0, tex_o.ctypes.data,
                w_o.ctypes.data)
    assert np.array_equal(full[0], tex_o) and full[1] == w_o[0]
    tr.close()


def test_noalloc_two_trainers_one_gpu():
    """a large and then a small model on one GPU share its scratch: each call's figures are its own"""
    big = Layout(1024, 768, [(256, 192, 4, False)], [16, 16], leak=0.0)
    lay = LAYOUTS["two_level"]
    tb = trainer(big, *data(big, 3))
    ts = trainer(lay, *data(lay, 4))
    rb, rs = tb.decode_error(), ts.decode_error()
    for _ in range(2):
        assert same(tb.decode_error_noalloc(), rb)
        assert same(ts.decode_error_noalloc(), rs)
    tb.close()
    ts.close()
