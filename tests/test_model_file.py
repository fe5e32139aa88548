"""The reference's model files (neural_block_textures_amd/model_file.py): a file the reference wrote
(tests/golden/ref_m1234_model.bin, v12) read field by field, decoded by the oracle and compared with
the reference's own decode of it (two crops and the per-channel sums of recon_003000_t*.png), and
write / read round trips of the v12 and v14 (DCT) layouts."""
import os

import numpy as np

from neural_block_textures_amd import model_file
from neural_block_textures_amd.trainer import PK_UV, Layout
from tests.helpers import GOLDEN, golden

MODEL = os.path.join(GOLDEN, "ref_m1234_model.bin")


def u8(v):
    return np.floor(np.clip(v, 0.0, 1.0).astype(np.float32) * np.float32(255.0) + 0.5).astype(np.uint8)


def test_read_reference_file():
    m = model_file.read(MODEL)
    lay = m.layout
    assert m.version == 12 and (lay.W, lay.H, lay.T) == (512, 512, 4)
    assert lay.levels == [(128, 128, 4, False), (64, 64, 4, False)] and lay.hidden == [36, 36] and lay.pos == [PK_UV]
    assert lay.leak == np.float32(0.01) and not lay.clamp_out and m.qat == 0 and m.dct is None
    assert m.z.size == 128 * 128 * 4 + 64 * 64 * 4 and m.p.size == lay.nparams == 2172


def test_oracle_decode_matches_reference_decode(orc):
    m = model_file.read(MODEL)
    ref = golden("ref_m1234_recon.npz")
    img = u8(orc.decode_full(m.layout, m.p, m.z)).reshape(512, 512, 12)
    for tag in ("a", "b"):
        y, x = ref[f"at_{tag}"]
        crop = img[y:y + 64, x:x + 64]
        d = np.abs(crop.astype(int) - ref[f"crop_{tag}"].astype(int))
        assert d.max() <= 1 and (d == 0).mean() > 0.999
    assert np.abs(img.reshape(-1, 12).astype(np.int64).sum(0) - ref["channel_sums"]).max() <= 64


def test_round_trip_v12(tmp_path):
    m = model_file.read(MODEL)
    p = str(tmp_path / "m.bin")
    model_file.write(p, m)
    assert open(p, "rb").read() == open(MODEL, "rb").read()


def test_round_trip_v14(tmp_path):
    lay = Layout(64, 48, [(64, 48, 2, True), (16, 12, 4, False)], [20, 12], T=1, pos=[PK_UV], leak=0.01)
    rng = np.random.default_rng(3)
    z = rng.normal(0, 0.3, lay.nz).astype(np.float32)
    z[:64 * 48 * 2] = 0.0
    nb = 8 * 6
    dct = {"N": 8, "dc_step": 4, "deadzone": 0, "q": [75, 30], "sym": rng.integers(-50, 50, nb * 2 * 64).astype(np.int16),
           "code": rng.integers(0, 16, nb * 2).astype(np.uint8)}
    m = model_file.ModelFile(14, lay, z, rng.normal(0, 0.2, lay.nparams).astype(np.float32), dct=dct)
    p = str(tmp_path / "d.bin")
    model_file.write(p, m)
    r = model_file.read(p)
    assert r.version == 14 and r.layout.levels == lay.levels and r.dct["q"] == [75, 30] and r.dct["deadzone"] == 0
    assert np.array_equal(r.dct["sym"], dct["sym"]) and np.array_equal(r.dct["code"], dct["code"])
    assert np.array_equal(r.z, z) and np.array_equal(r.p, m.p)


def test_post_hoc_8bit_decode_matches_reference(orc):
    """ntc_decode's default (--q8): the levels training left continuous on bitrate_stats' per-channel 8-bit
    grid; the oracle's decode of those values against the reference's recon_q_final_t*.png"""
    from neural_block_textures_amd import decode
    m = decode.load(MODEL)            # q8 by default
    raw = model_file.read(MODEL)
    assert not np.array_equal(m.z, raw.z)
    for (W, H, C, _), off in zip(m.layout.levels, m.layout.offsets):   # at most 256 values per channel
        lv = m.z[off:off + W * H * C].reshape(-1, C)
        assert max(np.unique(lv[:, c]).size for c in range(C)) <= 256
    ref = golden("ref_m1234_recon.npz")
    img = u8(orc.decode_full(m.layout, m.p, m.z)).reshape(512, 512, 12)
    for tag in ("a", "b"):
        y, x = ref[f"at_{tag}"]
        d = np.abs(img[y:y + 64, x:x + 64].astype(int) - ref[f"q_crop_{tag}"].astype(int))
        assert d.max() <= 1 and (d == 0).mean() > 0.999
    assert np.abs(img.reshape(-1, 12).astype(np.int64).sum(0) - ref["q_channel_sums"]).max() <= 64
