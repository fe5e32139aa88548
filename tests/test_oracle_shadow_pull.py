"""The oracle's --dct-shadow-pull (or_shadow_pull) against the reference's line, z += f * (zq - z) (main.cpp:4144),
compiled with the reference's flags, bit for bit, on inputs where a fused multiply-add and a separately rounded
multiply and add give different floats. Which of the two the reference's build produces is decided by its compiler;
this test pins the oracle (and, through tests/test_gpu_quant.py, the device's k_shadow_pull) to what it does."""
from fractions import Fraction

import numpy as np
import pytest

from oracle.oracle import have_reference, reference


def inputs(n=200000, seed=3):
    rng = np.random.default_rng(seed)
    z = rng.uniform(-1.2, 1.2, n).astype(np.float32)
    zq = (z + rng.normal(0, 0.05, n)).astype(np.float32)
    zq[: n // 4] = np.round(zq[: n // 4] * 8) / 8          # snapped values on a coarse grid, as a DCT plane's are
    return z, zq


def unfused(z, zq, f):
    d = (zq - z).astype(np.float32)
    return (z + (np.float32(f) * d).astype(np.float32)).astype(np.float32)


def exact_fused(z, zq, f):
    """z + f * (zq - z) with one rounding after the multiply-add (the subtraction rounded first)"""
    out = np.empty_like(z)
    ff = Fraction(float(np.float32(f)))
    for i in range(z.size):
        d = Fraction(float(np.float32(zq[i] - z[i])))
        out[i] = np.float32(float(Fraction(float(z[i])) + ff * d))   # float() of a Fraction rounds to nearest
    return out


@pytest.mark.parametrize("fast", [False, True], ids=["ref", "ref_fast"])
def test_shadow_pull_matches_reference_build(orc, fast):
    if not have_reference(fast=fast):
        pytest.skip("the reference build lives only where the reference tree is")
    L = reference(fast=fast).lib
    f = 0.01
    z, zq = inputs()
    a, b = z.copy(), z.copy()
    orc._shadow_pull(a.ctypes.data, zq.ctypes.data, z.size, f)
    L.ref_shadow_pull(b.ctypes.data, zq.ctypes.data, z.size, f)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # the inputs separate the two evaluation orders, so the equality above says which one the reference uses
    u = unfused(z, zq, f)
    sep = np.nonzero(u != b)[0]
    assert sep.size > 500
    # and it is the single-rounding multiply-add: checked exactly where the two orders differ, and on other values
    k = np.concatenate([sep, np.arange(1000)])
    assert np.array_equal(exact_fused(z[k], zq[k], f), b[k])


def test_shadow_pull_pull_of_one(orc):
    """F = 1 (--dct-shadow-reset) leaves the shadow equal to the snapped plane: z + (zq - z) = zq whenever zq - z is exact"""
    z, zq = inputs(2000, 5)
    a = z.copy()
    orc._shadow_pull(a.ctypes.data, zq.ctypes.data, z.size, 1.0)
    exact = (zq.astype(np.float64) - z.astype(np.float64)) == (zq - z).astype(np.float64)
    assert np.array_equal(a[exact], zq[exact])
