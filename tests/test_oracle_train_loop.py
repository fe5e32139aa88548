"""The oracle's training loop (or_train_iter) against the reference's own (ref_train_iter: main.cpp's
MlpTrainer / LatentTrainer / qat_search driven in the order of main.cpp:4121-4148, built from the
reference tree with GCC's default floating point). Every iteration's model and batch loss must be
identical bit for bit, through the switch to central differences (its Adam reset, main.cpp:4075-4084)
and with a --qat level (frozen in the latent step, searched every iteration).

This pins the loop itself - step order, the Adam step counters of both parameter vectors, the latent
step counter that keys the latent noise, the FD switch - beyond the per-function golden vectors."""
import ctypes as C

import numpy as np
import pytest

from oracle.oracle import Model, OrTrainCfg, OrTrainState, have_reference, model_of, reference

pytestmark = pytest.mark.skipif(not have_reference(), reason="the reference build exists only where the reference tree is")

F = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))

CASES = {
    # one bilinear level, ReLU (leak 0), uv
    "rgb_bilinear": (Model(32, 24, [(8, 6, 4, False)], [16, 16], leak=0.0), None),
    # two levels, bilinear + bilinear at ratios that are not powers of two, lv1local
    "two_level_lv1": (Model(30, 22, [(12, 9, 4, False), (5, 4, 2, False)], [12, 12], pos=[1], leak=0.01), None),
    # the material shape: 4 textures, --qat 2,1 on a nearest full-resolution level 0 + bilinear level 1
    "material_qat": (Model(24, 20, [(24, 20, 2, True), (6, 5, 4, False)], [16, 16], T=4, leak=0.01,
                           weights=[1.0, 2.0, 0.5, 1.5]), [2, 1]),
    # --qat on the only level: the latent step is skipped (main.cpp:4135)
    "qat_single_level": (Model(16, 16, [(16, 16, 2, True)], [12], T=1, leak=0.02), [3, 2]),
}


def init(lay, seed, qat_bits):
    rng = np.random.default_rng(seed)
    z = rng.normal(0, 0.3, lay.nz).astype(np.float32)
    if qat_bits:   # level 0 on its grid, as after the reference's qat initialisation
        n0 = lay.levels[0][0] * lay.levels[0][1] * lay.levels[0][2]
        z0 = z[:n0].reshape(-1, lay.levels[0][2])
        for c, b in enumerate(qat_bits):
            k = rng.integers(0, 1 << b, z0.shape[0])
            z0[:, c] = (-1.0 + 2.0 * k / ((1 << b) - 1)).astype(np.float32)
        z[:n0] = z0.ravel()
    p = rng.normal(0, 0.3, lay.nparams).astype(np.float32)
    tgt = (rng.integers(0, 256, lay.W * lay.H * lay.nout) / 255.0).astype(np.float32)
    return z, p, tgt


@pytest.mark.parametrize("name", list(CASES))
def test_train_loop_matches_reference(orc, name):
    ref = reference()
    lay, qat_bits = CASES[name]
    z, p, tgt = init(lay, 17, qat_bits)
    iters = 7
    cfg = OrTrainCfg()
    cfg.seed, cfg.mlp_pairs, cfg.mlp_batch, cfg.mlp_sigma, cfg.mlp_lr = 5, 8, 300, 0.02, 0.01
    cfg.lat_pairs, cfg.lat_sigma, cfg.lat_lr = 3, 0.05, 0.02
    cfg.fd_from, cfg.fd_h = 5, np.float32(1e-3)       # iterations 5..7 take central differences
    if qat_bits:
        cfg.qat = max(qat_bits)
        for c, b in enumerate(qat_bits):
            cfg.qat_ch[c] = b
    mc = model_of(lay)
    h = ref.lib.ref_train_create(C.byref(mc), C.byref(cfg), z.ctypes.data, p.ctypes.data, tgt.ctypes.data)
    assert h
    try:
        zo, po = z.copy(), p.copy()
        wm, wv = np.zeros_like(p), np.zeros_like(p)
        zm, zv = np.zeros_like(z), np.zeros_like(z)
        st = OrTrainState()
        st.z, st.p, st.wm, st.wv, st.zm, st.zv = F(zo), F(po), F(wm), F(wv), F(zm), F(zv)
        zr, pr = np.empty_like(z), np.empty_like(p)
        for it in range(1, iters + 1):
            l_ref = ref.lib.ref_train_iter(h, it, iters)
            l_or = orc.lib.or_train_iter(C.byref(mc), C.byref(cfg), C.byref(st), tgt.ctypes.data, it, iters)
            ref.lib.ref_train_get(h, zr.ctypes.data, pr.ctypes.data)
            assert l_or == l_ref, (it, l_or, l_ref)
            assert np.array_equal(po.view(np.uint32), pr.view(np.uint32)), f"weights differ after iteration {it}"
            assert np.array_equal(zo.view(np.uint32), zr.view(np.uint32)), f"latent differs after iteration {it}"
        assert not np.array_equal(po, p)                # the loop trained
        if len(lay.levels) > 1 or not qat_bits:
            assert not np.array_equal(zo[-lay.levels[-1][0] * lay.levels[-1][1] * lay.levels[-1][2]:],
                                      z[-lay.levels[-1][0] * lay.levels[-1][1] * lay.levels[-1][2]:])
        # the latent step ran once per iteration unless --qat froze the only level
        assert st.lat_step_no == (0 if (qat_bits and len(lay.levels) == 1) else iters)
    finally:
        ref.lib.ref_train_destroy(h)
