"""Host side of a DCT-coded level 0 (--dct-q), as the reference's main.cpp prepares it for the
backend: the 8x8 basis and zigzag handed over at init (ModelDesc.dct_basis / dct_zigzag), the
per-channel step tables and the --dct-lambda weights handed over by set_dct.

Every value is computed the way main.cpp computes it, in float32 where it uses float:
  basis   alpha(u) cos(pi (2x + 1) u / 16) in double, rounded once to float: the bit patterns of
          DCT_BASIS_BITS (main.cpp:657-668)
  A_k     1 / g_k with g_k = (14/64) 2^(0.6 k), rounded once to float: DCT_AK_BITS (main.cpp:670-681)
  zigzag  JPEG order: anti-diagonals s = u + v, even s with u decreasing (main.cpp:691-703)
  steps   Annex K Table K.1 scaled by the libjpeg quality scale and A_k (main.cpp:740-779)
"""
from __future__ import annotations

import math

import numpy as np

# JPEG Annex K Table K.1 (luminance), rows = vertical frequency u
JPEG_K1 = np.array([
    [16, 11, 10, 16, 24, 40, 51, 61], [12, 12, 14, 19, 26, 58, 60, 55],
    [14, 13, 16, 24, 40, 57, 69, 56], [14, 17, 22, 29, 51, 87, 80, 62],
    [18, 22, 37, 56, 68, 109, 103, 77], [24, 35, 55, 64, 81, 104, 113, 92],
    [49, 64, 78, 87, 103, 121, 120, 101], [72, 92, 95, 98, 112, 100, 103, 99],
], np.float32)


def basis() -> np.ndarray:
    """[u * 8 + x] float32"""
    b = np.zeros(64, np.float32)
    for u in range(8):
        a = math.sqrt(1.0 / 8.0) if u == 0 else math.sqrt(2.0 / 8.0)
        for x in range(8):
            b[u * 8 + x] = np.float32(a * math.cos(3.14159265358979323846 * (2 * x + 1) * u / 16.0))
    return b


def zigzag() -> np.ndarray:
    """zigzag position -> natural index u * 8 + v"""
    z = []
    for s in range(15):
        lo, hi = max(0, s - 7), min(7, s)
        us = range(lo, hi + 1) if s & 1 else range(hi, lo - 1, -1)
        z += [u * 8 + (s - u) for u in us]
    return np.array(z, np.int32)


def gain(k: int) -> float:
    return (14.0 / 64.0) * 2.0 ** (0.6 * k)


def ak() -> np.ndarray:
    return np.array([np.float32(1.0 / gain(k)) for k in range(16)], np.float32)


def quality_scale(q: int) -> np.float32:
    q = max(1, min(100, q))
    s = np.float32(5000.0) / np.float32(q) if q < 50 else np.float32(200.0) - np.float32(2.0) * np.float32(q)
    return np.float32(s * np.float32(1.0 / 100.0))


def steps(q: int, dc_step: int = 4) -> np.ndarray:
    """[16][64] integer steps of one channel: scale code k, natural index u * 8 + v; [k][0] = dc_step"""
    out = np.zeros((16, 64), np.int32)
    S, A = quality_scale(q), ak()
    for k in range(16):
        ls = np.float32(S * A[k])
        for u in range(8):
            for v in range(8):
                if u == 0 and v == 0:
                    out[k, 0] = dc_step
                elif q >= 100:
                    out[k, u * 8 + v] = 1
                else:
                    sf = np.float32(np.float32(JPEG_K1[u, v] * ls) + np.float32(0.5))
                    sf = min(max(sf, np.float32(1.0)), np.float32(1048576.0))
                    out[k, u * 8 + v] = max(1, int(sf))
    return out


def lambda_weights(lam: float, W: int, H: int, rate_es: bool, rate_trunc: bool):
    """(lam_t16[16], rate_scale): part B's lambda / (16 g_k^2) per scale code and part A's
    lambda / (16 * 65025 * W * H) (main.cpp:3534-3540, 2950-2951)"""
    t16 = np.array([np.float32(lam / (gain(k) * gain(k) * 16.0)) if rate_trunc else 0.0 for k in range(16)], np.float32)
    scale = np.float32(lam / (16.0 * 65025.0 * W * H)) if rate_es else np.float32(0.0)
    return t16, scale
