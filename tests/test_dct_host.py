"""The host side of a DCT-coded level 0 (neural_block_textures_amd/dct_host.py) against the oracle's
tables, which the known-answer tests pin to the reference's literals (DCT_BASIS_BITS, DCT_AK_BITS,
the JPEG zigzag and the step tables of --dct-selftest)."""
import numpy as np
import pytest

from neural_block_textures_amd import dct_host


def test_tables_bit_exact(orc):
    b, zz, ak = np.zeros(64, np.float32), np.zeros(64, np.int32), np.zeros(16, np.float32)
    orc.lib.or_dct_tables(b.ctypes.data, zz.ctypes.data, ak.ctypes.data)
    assert np.array_equal(dct_host.basis().view(np.uint32), b.view(np.uint32))
    assert np.array_equal(dct_host.zigzag(), zz)
    assert np.array_equal(dct_host.ak().view(np.uint32), ak.view(np.uint32))


@pytest.mark.parametrize("q", [1, 10, 25, 49, 50, 51, 75, 90, 99, 100])
@pytest.mark.parametrize("dc_step", [1, 4, 8])
def test_steps(orc, q, dc_step):
    st = np.zeros(1024, np.int32)
    orc.lib.or_dct_build_steps(q, dc_step, st.ctypes.data)
    assert np.array_equal(dct_host.steps(q, dc_step), st.reshape(16, 64))


def test_lambda_weights():
    # part B: lambda / (16 g_k^2) rounded once; part A: lambda / (16 * 65025 * W * H)
    t16, scale = dct_host.lambda_weights(0.5, 512, 512, True, True)
    g = lambda k: (14.0 / 64.0) * 2.0 ** (0.6 * k)
    assert t16[0] == np.float32(0.5 / (g(0) ** 2 * 16.0)) and t16.dtype == np.float32
    assert scale == np.float32(0.5 / (16.0 * 65025.0 * 512 * 512))
    t16, scale = dct_host.lambda_weights(0.5, 64, 64, False, False)
    assert not t16.any() and scale == 0
