"""The reference's bit-packed container (neural_block_textures_amd/ntcb.py) against containers the
reference itself wrote (tests/golden/ntcb_*.ntcb, from tests/golden/make_ntcb_fixture.py): every file
read and written back byte for byte; the writer, fed the model file the same run saved, produces the
reference's file byte for byte (palette, post-hoc grid, --qes grid and DCT levels, padding, --clamp);
the values the container holds decode (oracle) to the reference's own recon_q_final and to its
standalone decoder's output; corrupted files are refused with the reference's reasons; the fp16
rounding against the reference's own known answers (ntcb_selfcheck, main.cpp:2456-2470); the decoder's
post-hoc 8-bit rule applied to the run's model file gives exactly the container's values."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

from neural_block_textures_amd import dct_host, model_file, ntcb
from oracle.oracle import OrDct, OrLevel
from tests.helpers import GOLDEN, golden

CASES = ["qat4", "dct", "qes"]
LATENT_CELL = {"qat4": 0, "dct": 0, "qes": 8}


def raw(case):
    with open(os.path.join(GOLDEN, f"ntcb_{case}.ntcb"), "rb") as f:
        return f.read()


def u8(v):
    return np.floor(np.clip(v, 0.0, 1.0).astype(np.float32) * np.float32(255.0) + 0.5).astype(np.uint8)


def oracle_rgb8(orc, m: model_file.ModelFile) -> np.ndarray:
    """[T][src_h][src_w][3]: the oracle's decode of a model (a DCT level 0 reconstructed from its symbols)"""
    lay = m.layout
    z = m.z.copy()
    if m.dct:
        W0, H0, C0, _ = lay.levels[0]
        d = OrDct()
        d.C, d.BW, d.BH, d.dc_step, d.deadzone, d.lo_w16 = C0, W0 // 8, H0 // 8, m.dct["dc_step"], m.dct["deadzone"], 16
        steps = np.concatenate([dct_host.steps(q, m.dct["dc_step"]).reshape(-1) for q in m.dct["q"]]).astype(np.int32)
        code, sym = np.ascontiguousarray(m.dct["code"]), np.ascontiguousarray(m.dct["sym"])
        d.step = steps.ctypes.data_as(C.POINTER(C.c_int))
        d.code = code.ctypes.data_as(C.POINTER(C.c_uint8))
        d.sym = sym.ctypes.data_as(C.POINTER(C.c_int16))
        zq = np.zeros(W0 * H0 * C0, np.float32)
        orc._dct_recon_level0(C.byref(d), C.byref(OrLevel(W0, H0, C0, 1, 0)), zq.ctypes.data, None)
        z[:zq.size] = zq
    img = u8(orc.decode_full(lay, m.p, z)).reshape(lay.H, lay.W, lay.T, 3)
    return img.transpose(2, 0, 1, 3)[:, :m.size[3], :m.size[2]]


@pytest.mark.parametrize("case", CASES)
def test_read_and_write_back(case):
    b = raw(case)
    n = ntcb.parse(b)
    assert ntcb.to_bytes(n) == b
    assert n.latent_cell == LATENT_CELL[case] and n.version == 2


def test_fields_of_the_reference_files():
    q = ntcb.parse(raw("qat4"))
    assert (q.img_w, q.img_h, q.src_w, q.src_h, q.T, q.hidden, q.pos, q.clamp) == (64, 64, 64, 64, 4, [16, 16], "uv", False)
    assert [(L.mode, L.bits) for L in q.levels] == [(2, [2, 2]), (0, [8] * 4)]
    assert all(np.array_equal(pal, ntcb.qat_palette(2)) for pal in q.levels[0].palette)
    d = ntcb.parse(raw("dct"))
    L0 = d.levels[0]
    assert (L0.mode, L0.q, L0.dc_step, d.dct_block) == (3, [50], 4, 8) and L0.sym.size == 64 * 64 and L0.code.size == 64
    s = ntcb.parse(raw("qes"))
    assert (s.img_w, s.img_h, s.src_w, s.src_h, s.clamp) == (64, 48, 60, 44, True)
    assert [(L.mode, L.bits[0]) for L in s.levels] == [(1, 6), (1, 6)]


@pytest.mark.parametrize("case", CASES)
def test_writer_from_the_runs_model_file(case):
    """ntcb_write's mode choice, grid ranges and indices from the state the run saved"""
    m = model_file.read(os.path.join(GOLDEN, f"ntcb_{case}_model.bin"))
    n = ntcb.from_model_file(m, latent_cell=LATENT_CELL[case])
    assert ntcb.to_bytes(n) == raw(case)


@pytest.mark.parametrize("case", CASES)
def test_values_decode_to_the_references_images(orc, case):
    n = ntcb.parse(raw(case))
    m = n.to_model_file()
    mf = model_file.read(os.path.join(GOLDEN, f"ntcb_{case}_model.bin"))
    # palette / --qes levels hold exactly the values the run saved; DCT symbols and codes likewise
    lay = m.layout
    for l, ((W, H, Cc, _), off) in enumerate(zip(lay.levels, lay.offsets)):
        if n.levels[l].mode in (1, 2):
            assert np.array_equal(m.z[off:off + W * H * Cc], mf.z[off:off + W * H * Cc])
    if m.dct:
        assert np.array_equal(m.dct["sym"], mf.dct["sym"]) and np.array_equal(m.dct["code"], mf.dct["code"])
    img = oracle_rgb8(orc, m)
    ref = golden(f"ntcb_{case}_images.npz")
    for k in ("recon_q_final", "ntc_decode"):
        assert img.shape == ref[k].shape
        d = np.abs(img.astype(int) - ref[k].astype(int))
        assert d.max() <= 1 and (d == 0).mean() > 0.999, (k, d.max(), (d == 0).mean())


def refit(b: bytearray) -> bytes:
    struct.pack_into("<I", b, 28, ntcb.file_hash(bytes(b)))
    return bytes(b)


def refused(b: bytes, why: str):
    with pytest.raises(ValueError, match=why):
        ntcb.parse(b)


def test_refusals():
    """the reader's checks (NTCB_NOTES section 3(f), main.cpp:2540-2618, 2762-2846)"""
    b = raw("qat4")
    n = ntcb.parse(b)
    H = struct.unpack_from("<H", b, 6)[0]
    refused(b[:7], "shorter than 8 bytes")
    refused(b"ntcX" + b[4:], "bad magic")
    refused(b[:-1], "file_bytes")
    refused(b + b"\0", "file_bytes")
    x = bytearray(b)
    x[H + 20] ^= 0x10
    refused(bytes(x), "hash mismatch")
    x = bytearray(b)                                  # version 3
    struct.pack_into("<H", x, 4, 3)
    refused(refit(x), "ntcb version 3")
    x = bytearray(b)                                  # the level-0 sync marker
    x[H + 8] ^= 0x01
    refused(refit(x), "sync marker mismatch before level 0 body")
    x = bytearray(b)                                  # a coded section
    x[H + 1] = 1
    refused(refit(x), "coded sections")
    x = bytearray(b)                                  # reserved header byte
    x[39] = 1
    refused(refit(x), "header field out of range")
    x = bytearray(b)                                  # 5 textures
    x[34] = 5
    refused(refit(x), "header field out of range")
    # a level record with a bad mode, and a container whose sections do not fit
    off = 52 + n.T + 2 * len(n.hidden) + 2 + len(n.pos)
    x = bytearray(b)
    x[off + 11] = 4
    refused(refit(x), "bad dims")
    x = bytearray(b[:-40])
    struct.pack_into("<I", x, 24, len(x))
    refused(refit(x), "sections need at least")
    # DCT: a run past the 63 AC positions is refused, as is a bad quality
    d = raw("dct")
    nd = ntcb.parse(d)
    x = bytearray(d)
    qoff = 52 + nd.T + 2 * len(nd.hidden) + 2 + len(nd.pos) + 12 + 1 + 2
    x[qoff] = 101
    refused(refit(x), "dct quality 101")


def test_writer_refusals():
    m = model_file.read(os.path.join(GOLDEN, "ntcb_qat4_model.bin"))
    bad = model_file.read(os.path.join(GOLDEN, "ntcb_qat4_model.bin"))
    bad.p = bad.p.copy()
    bad.p[3] = np.float32(0.1)                        # not an fp16 value
    with pytest.raises(ValueError, match="not an fp16 value"):
        ntcb.from_model_file(bad)
    off = m.z.copy()
    off[0] = np.float32(0.3)                          # a level-0 value off its --qat grid
    bad = model_file.read(os.path.join(GOLDEN, "ntcb_qat4_model.bin"))
    bad.z = off
    with pytest.raises(ValueError, match="off its --qat grid"):
        ntcb.from_model_file(bad)
    with pytest.raises(ValueError, match="2..12"):
        ntcb.from_model_file(m, qbits=13)
    with pytest.raises(ValueError, match="latent_cell"):
        ntcb.from_model_file(m, latent_cell=256)


def test_fp16_rounding_known_answers():
    """ntcb_selfcheck's cases (round to nearest even, the smallest denormal, overflow) and every finite
    half pattern through float and back"""
    def h(x):
        return int(np.float32(x).astype(np.float16).view(np.uint16))
    assert (h(1.0), h(-2.0), h(65504.0), h(5.9604645e-8), h(2.9802322e-8), h(1.00048828), h(1.00073242)) == \
        (0x3C00, 0xC000, 0x7BFF, 0x0001, 0x0000, 0x3C00, 0x3C01)
    with pytest.raises(ValueError):
        ntcb.round_fp16(np.array([65520.0], np.float32))          # rounds to 2^16: no fp16 value
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    pats = pats[(pats & 0x7C00) != 0x7C00]
    f = pats.view(np.float16).astype(np.float32)
    assert np.array_equal(ntcb.f16_bits(f), pats)
    assert np.array_equal(ntcb.round_fp16(f), f)


def test_sync_values_distinct():
    """every (level, channel) marker of a kind differs (main.cpp:2373-2378)"""
    for base in (ntcb.SYNC_LEVEL, ntcb.SYNC_CHANNEL, ntcb.SYNC_MLP, ntcb.SYNC_END):
        v = {ntcb.sync_value(base, l, c) for l in range(4) for c in range(4 if base == ntcb.SYNC_CHANNEL else 1)}
        assert len(v) == (16 if base == ntcb.SYNC_CHANNEL else 4)


@pytest.mark.parametrize("case", CASES)
def test_post_hoc_grid_of_the_model_file_is_the_containers(case):
    """decode.load's --q8 rule on the run's model file gives exactly the values its container holds"""
    from neural_block_textures_amd import decode
    m = decode.load(os.path.join(GOLDEN, f"ntcb_{case}_model.bin"))
    n = ntcb.parse(raw(case)).to_model_file()
    assert np.array_equal(m.z, n.z)
