"""Layouts and helpers of the GPU parity tests (HIP path through the C ABI against the oracle)."""
from __future__ import annotations

import os
import sys

import numpy as np

from neural_block_textures_amd import synth
from neural_block_textures_amd.trainer import PK_LV1LOCAL, PK_UV, Layout, Trainer

# One layout per compiled MLP shape, at sizes the oracle finishes in seconds, plus one that runs
# through the runtime-shaped kernels (3 levels, lv1local, clamp output, ratios not powers of 2).
LAYOUTS = {
    "rgb_16x2": Layout(64, 64, [(16, 16, 4, False)], [16, 16], leak=0.0),
    "rgb_24x2": Layout(48, 48, [(12, 12, 4, False)], [24, 24], leak=0.01),
    "two_level": Layout(96, 64, [(24, 16, 8, False), (6, 4, 4, False)], [32, 32], leak=0.0),
    "material": Layout(48, 40, [(48, 40, 2, True), (12, 10, 4, False)], [32, 32], T=4, leak=0.01,
                       weights=[1.0, 2.0, 0.5, 1.5]),
    "dct_plane": Layout(64, 48, [(64, 48, 1, True), (16, 12, 4, False)], [32, 32], leak=0.01),
    "large": Layout(48, 48, [(24, 24, 4, False), (6, 6, 8, False)], [64, 64], T=4, leak=0.0),
    "runtime": Layout(50, 38, [(13, 10, 3, True), (5, 4, 4, False), (3, 3, 2, False)], [20, 12], T=2,
                      pos=[PK_LV1LOCAL, PK_UV], leak=0.02, clamp_out=True, weights=[1.0, 3.0]),
    # the reference's published runs (README.md:358, 382, 531): selector plane, nearest block latent,
    # lv1local, hidden widths that pad the matrix tiles (36 -> 48, 27 -> 32)
    "chief1_36": Layout(64, 48, [(64, 48, 1, True), (16, 12, 2, True)], [36, 36], pos=[PK_LV1LOCAL], leak=1 / 1024),
    "mat_qat_36": Layout(48, 40, [(48, 40, 2, True), (12, 10, 4, True)], [36, 36], T=4, pos=[PK_LV1LOCAL],
                         leak=1 / 1024, weights=[1.0, 2.0, 0.5, 1.5]),
    "image3_27": Layout(64, 48, [(64, 48, 1, True), (8, 6, 4, False)], [27, 27], pos=[PK_LV1LOCAL], leak=1 / 1024),
    # README.md:620's 17-wide DCT decoder: 2 hidden tiles, the second with one unit
    "dct_17": Layout(64, 48, [(64, 48, 1, True), (16, 12, 4, False)], [17, 17], pos=[PK_LV1LOCAL], leak=1 / 1024),
    # README.md:991's 3-texture material (9 outputs) and README.md:298's 4-texture --qat 2 with a 4-channel block
    "run8x3": Layout(64, 48, [(32, 24, 8, False), (16, 12, 4, False)], [24, 24], T=3, weights=[1.0, 1.0, 0.5]),
    "mat_qat1x4_36": Layout(48, 40, [(48, 40, 1, True), (12, 10, 4, True)], [36, 36], T=4, pos=[PK_LV1LOCAL],
                            leak=1 / 1024),
    # shapes the library does not list: kernels specialised at init (hipRTC); VALU only, and with the
    # matrix cores
    "jit_valu_7": Layout(64, 48, [(16, 12, 4, False)], [7, 7], leak=0.01),
    "jit_mfma_28": Layout(48, 40, [(48, 40, 2, True), (12, 10, 4, False)], [28, 28], T=4, pos=[PK_LV1LOCAL], leak=0.01,
                          weights=[1.0, 0.5, 2.0, 1.0]),
}
# the same layouts with every stage forced onto the VALU kernels (ntc_trainer_set_matrix_cores(0))
for _name in ("material", "chief1_36"):
    _lay = Layout(**{k: getattr(LAYOUTS[_name], k) for k in LAYOUTS[_name].__dataclass_fields__})
    _lay.valu_only = True
    LAYOUTS[_name + "_valu"] = _lay
# "runtime" (hidden widths 20, 12) on the runtime-shaped kernels, and the same model on the kernels
# specialised at init for its widths (FixedShapeW)
LAYOUTS["jit_widths"] = Layout(**{k: getattr(LAYOUTS["runtime"], k) for k in LAYOUTS["runtime"].__dataclass_fields__})
LAYOUTS["runtime"].runtime_kernels = True


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def data(layout: Layout, seed: int, zscale=0.4):
    rng = np.random.default_rng(seed)
    z = rng.normal(0, zscale, layout.nz).astype(np.float32)
    p = synth.init_model(layout, seed)[1]
    p = (p + rng.normal(0, 0.05, p.size)).astype(np.float32)   # nonzero biases
    tgt = (rng.integers(0, 256, layout.W * layout.H * layout.nout).astype(np.float32) / np.float32(255.0))
    return z, p, tgt.astype(np.float32)


def trainer(layout: Layout, z, p, tgt, *, max_pairs=64, max_batch=4096, seed=5, **kw):
    tr = Trainer()
    d = Trainer.model_desc(layout, max_pairs=max_pairs, max_batch=max_batch, seed=seed, **kw)
    if getattr(layout, "runtime_kernels", False):   # NTC_HIP_JIT=0: the runtime-shaped kernels, not specialised ones
        old = os.environ.get("NTC_HIP_JIT")
        os.environ["NTC_HIP_JIT"] = "0"
        try:
            tr.init(d, z, p, tgt, layout)
        finally:
            if old is None:
                del os.environ["NTC_HIP_JIT"]
            else:
                os.environ["NTC_HIP_JIT"] = old
    else:
        tr.init(d, z, p, tgt, layout)
    if getattr(layout, "valu_only", False):
        tr.set_matrix_cores(False)
    return tr


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.abs(a - b) / np.maximum(np.abs(b), 1e-300)
