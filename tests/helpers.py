"""Shared test helpers: fixture loading and the layouts the parity tests run."""
from __future__ import annotations

import os

import numpy as np

from neural_block_textures_amd.trainer import Layout

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def layout_of(fx: dict) -> Layout:
    lv = [tuple(int(x) for x in row[:3]) + (bool(row[3]),) for row in fx["levels"]]
    return Layout(int(fx["W"]), int(fx["H"]), lv, [int(h) for h in fx["hidden"]], T=int(fx["T"]),
                  pos=[int(q) for q in fx["pos"]], leak=float(fx["leak"]), clamp_out=bool(int(fx["clamp_out"])),
                  weights=[float(w) for w in fx["weights"]])


def model_data(layout: Layout, seed: int, zscale=0.4, pscale=0.35):
    rng = np.random.default_rng(seed)
    z = rng.normal(0, zscale, layout.nz).astype(np.float32)
    p = rng.normal(0, pscale, layout.nparams).astype(np.float32)
    tgt = (rng.integers(0, 256, layout.W * layout.H * layout.nout).astype(np.float32) / np.float32(255.0)).astype(np.float32)
    return z, p, tgt
