"""Latent steps whose pairs run in groups (ntc_trainer_set_lat_group): the gradient, the Adam step and the DCT rate
pass's figures equal the ungrouped step's bit for bit. The groups add their pairs to every texel's gradient after the
previous groups' pairs, in the reference's pair order (LatentTrainer::step_impl, main.cpp:1990-2037), and the shadow
moves only after the last group; the step then holds one group's Gaussians and per-pixel differences at a time."""
import numpy as np
import pytest

from neural_block_textures_amd import synth
from tests.gpu_common import LAYOUTS, HostDct, data, dct_tables, say, trainer

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name,K,G", [("two_level", 7, 3), ("material", 5, 2), ("rgb_16x2", 9, 1)])
def test_grouped_latent_steps_equal(orc, name, K, G):
    lay = LAYOUTS[name]
    say("latent groups", name, K, G)
    z, p, tgt = data(lay, 21)
    kw = {}
    if name == "material":   # --qat 2,2: level 0 outside the perturbation mask
        grid = synth.qat_grid()
        n0 = lay.levels[0][0] * lay.levels[0][1] * lay.levels[0][2]
        lv0 = z[:n0].reshape(-1, lay.levels[0][2])
        for c in range(lay.levels[0][2]):
            lv0[:, c] = synth.qat_snap(lv0[:, c], 2, grid)
        z[:n0] = lv0.reshape(-1)
        kw = dict(qat_bits=[2, 2], qat_grid=grid)
    a = trainer(lay, z, p, tgt, **kw)
    b = trainer(lay, z, p, tgt, **kw)
    b.set_lat_group(G)
    for it in (1, 2, 3):
        a.lat_step(it, 0.05, 0.02, K)
        b.lat_step(it, 0.05, 0.02, K)
        assert np.array_equal(bits(a.debug_last_zgrad()), bits(b.debug_last_zgrad())), it
        assert np.array_equal(bits(a.download_model()[0]), bits(b.download_model()[0])), it
    # the grouped trainer's per-pixel differences are its last group's: the ungrouped step's last rows
    last = K - (K - 1) // G * G
    da, db = a.debug_last_dpix().reshape(-1), b.debug_last_dpix().reshape(-1)
    assert db.size == last * lay.W * lay.H and np.array_equal(bits(db), bits(da[da.size - db.size:]))
    a.close()
    b.close()


def test_drawn_ahead_gaussians_follow_the_pair_count(orc):
    """A step that runs as one group draws the next step's latent Gaussians (step + 1, the same pair count) in its last
    gather launch. Steps whose pair count changes draw their own instead. Against a trainer that never draws ahead
    (one pair per group), every step's gradient and latent are equal bit for bit, across both kinds of step."""
    lay = LAYOUTS["two_level"]
    say("latent draw-ahead", "two_level")
    z, p, tgt = data(lay, 5)
    a = trainer(lay, z, p, tgt)
    b = trainer(lay, z, p, tgt)
    b.set_lat_group(1)
    for it, K in enumerate((4, 4, 6, 6, 6, 3, 4), start=1):
        a.lat_step(it, 0.05, 0.02, K)
        b.lat_step(it, 0.05, 0.02, K)
        assert np.array_equal(bits(a.debug_last_zgrad()), bits(b.debug_last_zgrad())), (it, K)
        assert np.array_equal(bits(a.download_model()[0]), bits(b.download_model()[0])), (it, K)
    a.close()
    b.close()


def test_grouped_latent_step_dct_rate(orc):
    """a live --dct-q level 0 with the rate term: every group's rate pass writes its pairs' bit differences, so the
    step's hit count, the last pair's differences and the gradient are the ungrouped step's"""
    lay = LAYOUTS["dct_plane"]
    z, p, tgt = data(lay, 14, zscale=0.7)
    basis, zz = dct_tables(orc)
    n0 = lay.levels[0][0] * lay.levels[0][1]
    trs = []
    for G in (0, 2):
        tr = trainer(lay, z, p, tgt, dct={"C": 1, "dc_step": 4, "q": [50]}, dct_basis=basis, dct_zigzag=zz)
        H = HostDct(orc, lay, [50], lam=0.5, rate="both")
        zd, _ = tr.download_model()
        H.probe(lay, p, np.concatenate([zd[:n0], z[n0:]]))
        H.snap(zd)
        tr.set_dct(H.desc(), H.code, H.sym, H.steps)
        tr.set_lat_group(G)
        trs.append(tr)
    K = 5
    for it in (1, 2):
        for tr in trs:
            tr.lat_step(it, 0.05, 0.02, K)
        ra, rb = trs[0].download_dct_rate(), trs[1].download_dct_rate()
        say("dct rate, grouped in 2: hits", rb[4], "of", rb[5])
        assert ra[4] == rb[4] and ra[5] == rb[5] and np.array_equal(ra[1], rb[1]) and np.array_equal(ra[0], rb[0])
        assert np.array_equal(bits(trs[0].debug_last_zgrad()), bits(trs[1].debug_last_zgrad()))
        assert np.array_equal(bits(trs[0].download_zq()), bits(trs[1].download_zq()))
    for tr in trs:
        tr.close()
