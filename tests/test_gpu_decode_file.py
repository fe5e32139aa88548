"""GPU decode of model files (neural_block_textures_amd/decode.py): the reference's own v12 file decoded
on the device to 8 bits, against the reference's decode of it (crops and channel sums of
recon_003000_t*.png) and against the oracle's decode; a v14 file (DCT-coded level 0) reconstructed and
decoded on the device against the oracle's reconstruction and decode."""
import ctypes as C
import os

import numpy as np
import pytest

from neural_block_textures_amd import model_file
from neural_block_textures_amd.decode import trainer_for
from neural_block_textures_amd.trainer import PK_UV, Layout
from oracle.oracle import OrDct, OrLevel
from tests.gpu_common import say
from tests.helpers import GOLDEN, golden

pytestmark = pytest.mark.gpu


def u8(v):
    return np.floor(np.clip(v, 0.0, 1.0).astype(np.float32) * np.float32(255.0) + 0.5).astype(np.uint8)


def test_decode_reference_file(orc):
    m = model_file.read(os.path.join(GOLDEN, "ref_m1234_model.bin"))
    say("decode ref_m1234_model.bin", m.layout.W, m.layout.H, m.layout.T)
    tr = trainer_for(m)
    img = tr.decode_rgb8().reshape(512, 512, 12)
    tr.close()
    ref = golden("ref_m1234_recon.npz")
    for tag in ("a", "b"):
        y, x = ref[f"at_{tag}"]
        d = np.abs(img[y:y + 64, x:x + 64].astype(int) - ref[f"crop_{tag}"].astype(int))
        assert d.max() <= 1 and (d == 0).mean() > 0.999
    assert np.abs(img.reshape(-1, 12).astype(np.int64).sum(0) - ref["channel_sums"]).max() <= 64
    o = u8(orc.decode_full(m.layout, m.p, m.z)).reshape(512, 512, 12)
    d = np.abs(img.astype(int) - o.astype(int))
    say("device vs oracle: max", d.max(), "exact", (d == 0).mean())
    assert d.max() <= 1 and (d == 0).mean() > 0.9999


def test_decode_dct_file(orc, tmp_path):
    lay = Layout(64, 48, [(64, 48, 2, True), (16, 12, 4, False)], [20, 12], T=1, pos=[PK_UV], leak=0.01)
    rng = np.random.default_rng(5)
    nb, C0 = 8 * 6, 2
    q = [75, 30]
    from neural_block_textures_amd import dct_host
    steps = np.concatenate([dct_host.steps(v, 4).reshape(-1) for v in q])
    sym = (rng.integers(-3, 4, nb * C0 * 64) * (rng.random(nb * C0 * 64) < 0.3)).astype(np.int16)
    sym[::64] = rng.integers(-60, 60, nb * C0).astype(np.int16)          # the DC symbols
    code = rng.integers(0, 16, nb * C0).astype(np.uint8)
    z = rng.normal(0, 0.3, lay.nz).astype(np.float32)
    z[:64 * 48 * C0] = 0.0
    p = (rng.normal(0, 0.3, lay.nparams)).astype(np.float32)
    m = model_file.ModelFile(14, lay, z, p, dct={"N": 8, "dc_step": 4, "deadzone": 0, "q": q, "sym": sym, "code": code})
    path = str(tmp_path / "d.bin")
    model_file.write(path, m)
    r = model_file.read(path)
    tr = trainer_for(r)
    img = tr.decode_rgb8()
    tr.close()
    # the oracle: level 0 reconstructed from the symbols, then the decode
    d = OrDct()
    d.C, d.BW, d.BH, d.dc_step, d.deadzone, d.lo_w16 = C0, 8, 6, 4, 0, 16
    d.step = steps.ctypes.data_as(C.POINTER(C.c_int))
    d.code = code.ctypes.data_as(C.POINTER(C.c_uint8))
    d.sym = sym.ctypes.data_as(C.POINTER(C.c_int16))
    zq = np.zeros(64 * 48 * C0, np.float32)
    orc._dct_recon_level0(C.byref(d), C.byref(OrLevel(64, 48, C0, 1, 0)), zq.ctypes.data, None)
    zz = z.copy()
    zz[:zq.size] = zq
    o = u8(orc.decode_full(lay, p, zz))
    dd = np.abs(img.astype(int) - o.astype(int))
    assert dd.max() <= 1 and (dd == 0).mean() > 0.999
