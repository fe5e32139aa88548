"""GPU decode of the reference's bit-packed containers (tests/golden/ntcb_*.ntcb, written by the reference's
own program): each container read (neural_block_textures_amd/ntcb.py), its model installed on the device
(neural_block_textures_amd/decode.py) and decoded to 8 bits there, against the oracle's decode of the
same values, the reference trainer's recon_q_final and the reference's standalone decoder's output."""
import os

import numpy as np
import pytest

from neural_block_textures_amd import decode, ntcb
from tests.gpu_common import say
from tests.helpers import GOLDEN, golden
from tests.test_ntcb import CASES, oracle_rgb8

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", CASES)
def test_decode_container(orc, case):
    path = os.path.join(GOLDEN, f"ntcb_{case}.ntcb")
    say("decode container", case)
    m = decode.load(path)
    lay = m.layout
    tr = decode.trainer_for(m)
    rgb = tr.decode_rgb8().reshape(lay.H, lay.W, lay.T, 3).transpose(2, 0, 1, 3)
    tr.close()
    n = ntcb.read(path)
    img = rgb[:, :n.src_h, :n.src_w]
    o = oracle_rgb8(orc, m)
    d = np.abs(img.astype(int) - o.astype(int))
    say("device vs oracle: max", d.max(), "equal", (d == 0).mean())
    assert d.max() <= 1 and (d == 0).mean() > 0.9999
    ref = golden(f"ntcb_{case}_images.npz")
    for k in ("recon_q_final", "ntc_decode"):
        d = np.abs(img.astype(int) - ref[k].astype(int))
        say("device vs", k, "max", d.max(), "equal", (d == 0).mean())
        assert d.max() <= 1 and (d == 0).mean() > 0.999
