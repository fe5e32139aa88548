"""The C ABI of libntc_hip.so without a GPU: every symbol include/ntc_hip.h declares is exported
(and so are the C++ ntc_cuda::Trainer methods main.cpp links against), the ctypes mirrors have
the compiled layouts, and models outside the envelope are refused with the reference's reasons
before any device call."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from neural_block_textures_amd import trainer as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "ntc_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ntc_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = T.library()
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_cpp_trainer_symbols_for_main_cpp():
    out = subprocess.run(["nm", "-DC", "--defined-only", T.LIB_PATH], capture_output=True, text=True).stdout
    for m in ["init", "banner", "upload_model", "download_model", "set_qes", "snap_latent", "shadow_pull", "download_zq",
              "set_dct", "download_dct", "download_dct_rate", "mlp_step", "mlp_step_fd", "reset_mlp_adam", "mlp_stats",
              "lat_step", "qat_search", "decode_full", "debug_last_batch", "debug_last_dl", "debug_last_zgrad"]:
        assert re.search(rf"ntc_cuda::Trainer::{m}(\[abi:cxx11\])?\(", out), m
    assert "ntc_cuda::Trainer::Trainer()" in out and "ntc_cuda::Trainer::~Trainer()" in out


@pytest.mark.parametrize("name,cls", [("ntc_model_desc", T.ModelDesc), ("ntc_qes_desc", T.QesDesc),
                                      ("ntc_dct_desc", T.DctDesc), ("ntc_level_desc", T.LevelDesc),
                                      ("ntc_print_stats", T.PrintStats)])
def test_struct_layouts(name, cls):
    assert T.library().ntc_abi_sizeof(name.encode()) == C.sizeof(cls)


def _init(layout, **kw):
    tr = T.Trainer()
    d = T.Trainer.model_desc(layout, **kw)
    z = np.zeros(max(layout.nz, 1), np.float32)
    p = np.zeros(max(layout.nparams, 1), np.float32)
    tgt = np.zeros(layout.W * layout.H * layout.nout, np.float32)
    return tr, d, z, p, tgt


@pytest.mark.parametrize("mutate,reason", [
    (lambda d: setattr(d, "nlev", 0), "bad level count"),
    (lambda d: setattr(d, "nlev", 4), "bad level count"),
    (lambda d: d.hidden.__setitem__(0, 65), "at most 64 units per layer"),
    (lambda d: setattr(d, "nout", 13), "too many MLP outputs"),
    (lambda d: setattr(d, "max_pairs", 0), "bad pair / batch counts"),
    (lambda d: setattr(d, "nin", 7), "nin differs"),
    (lambda d: d.qes_bits.__setitem__(0, 13), "--qes bits out of range"),
    (lambda d: setattr(d, "W", 1 << 15) or setattr(d, "H", 1 << 13), "images below 2^28 pixels"),
])
def test_envelope_refusals(mutate, reason):
    lay = T.Layout(64, 64, [(16, 16, 4, False)], [24, 24])
    tr, d, z, p, tgt = _init(lay)
    mutate(d)
    with pytest.raises(ValueError, match=re.escape(reason)):
        tr.init(d, z, p, tgt)


def test_dct_and_qat_refusals():
    lay = T.Layout(64, 64, [(64, 64, 5, True)], [16])
    tr, d, z, p, tgt = _init(lay)
    d.dct, d.dct_C, d.dct_N = 1, 5, 8
    with pytest.raises(ValueError, match="1..4 channels"):
        tr.init(d, z, p, tgt)
    lay = T.Layout(64, 64, [(32, 32, 2, False)], [16])
    tr, d, z, p, tgt = _init(lay)
    d.dct, d.dct_C, d.dct_N = 1, 2, 8
    with pytest.raises(ValueError, match="full-resolution nearest"):
        tr.init(d, z, p, tgt)
    tr, d, z, p, tgt = _init(lay)
    d.qat, d.qat_bits[0], d.qat_bits[1] = 2, 2, 2
    with pytest.raises(ValueError, match="grid table"):
        tr.init(d, z, p, tgt)
