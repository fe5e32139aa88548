"""End-to-end: a short training run on the device against the oracle's CPU loop (final PSNR
within 0.05 dB, the task's bar), and the benchmark workloads at their full sizes through
size-independent properties (an unperturbed population has exactly zero loss differences and
equal member losses; member losses of sampled pairs match the oracle on the device's own
minibatch; frozen levels get exactly zero gradient; every --qat value stays on its grid)."""
import ctypes as C
import time

import numpy as np
import pytest

from neural_block_textures_amd import synth
from neural_block_textures_amd.configs import workloads
from neural_block_textures_amd.trainer import Layout
from oracle.oracle import OrTrainCfg, OrTrainState, have_reference, model_of, oracle, reference
from tests.gpu_common import HostDct, dct_tables, rel, say, trainer

pytestmark = pytest.mark.gpu


def psnr(img, tgt, T):
    a = np.rint(np.clip(img, 0, 1) * 255.0)
    b = np.rint(np.clip(tgt, 0, 1) * 255.0)
    mse = ((a - b) ** 2).mean()
    return 10 * np.log10(255.0 ** 2 / mse) if mse > 0 else 100.0


@pytest.mark.parametrize("qat", [False, True])
def test_trajectory_psnr(orc, qat):
    if qat:
        lay = Layout(64, 64, [(64, 64, 2, True), (16, 16, 4, False)], [32, 32], T=4, leak=0.01)
        bits = [2, 2]
        maps = synth.material(21, 64, 64)
    else:
        lay = Layout(64, 64, [(16, 16, 4, False)], [16, 16], leak=0.0)
        bits = None
        maps = [synth.rgb_texture(21, 64, 64)]
    tgt = synth.target_from_maps(maps)
    z, p = synth.init_model(lay, 21, qat_bits=bits)
    N, M, iters, seed = 16, 2048, 25, 3
    say("trajectory qat" if qat else "trajectory", iters)
    tr = trainer(lay, z, p, tgt, max_pairs=N, max_batch=M, seed=seed, qat_bits=bits,
                 qat_grid=synth.qat_grid() if qat else None)
    cfg = OrTrainCfg()
    cfg.seed, cfg.mlp_pairs, cfg.mlp_batch, cfg.mlp_sigma, cfg.mlp_lr = seed, N, M, 0.02, 0.005
    cfg.lat_pairs, cfg.lat_sigma, cfg.lat_lr, cfg.fd_from, cfg.fd_h = 4, 0.05, 0.02, iters - 4, 1e-3
    if qat:
        cfg.qat = 2
        cfg.qat_ch[0], cfg.qat_ch[1] = 2, 2
    zo, po = z.copy(), p.copy()
    wm, wv = np.zeros_like(p), np.zeros_like(p)
    zm, zv = np.zeros_like(z), np.zeros_like(z)
    st = OrTrainState()
    F = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    st.z, st.p, st.wm, st.wv, st.zm, st.zv = F(zo), F(po), F(wm), F(wv), F(zm), F(zv)
    mc = model_of(lay)
    for it in range(1, iters + 1):
        if it == cfg.fd_from:
            tr.reset_mlp_adam()
        if it >= cfg.fd_from:
            tr.mlp_step_fd(it, np.float32(1e-3), 0.005, M)
        else:
            tr.mlp_step(it, 0.02, 0.005, N, M)
        tr.lat_step(it, 0.05, 0.02, 4)
        if qat:
            tr.qat_search()
        orc.lib.or_train_iter(C.byref(mc), C.byref(cfg), C.byref(st), tgt.ctypes.data, it, iters)
    zg, pg = tr.download_model()
    ps_gpu = psnr(tr.decode_full(), tgt, lay.T)
    ps_cpu = psnr(orc.decode_full(lay, po, zo), tgt, lay.T)
    ps_0 = psnr(orc.decode_full(lay, p, z), tgt, lay.T)
    say(f"psnr start {ps_0:.3f} gpu {ps_gpu:.3f} cpu {ps_cpu:.3f}")
    assert ps_cpu > ps_0 + 0.5          # training moved
    assert abs(ps_gpu - ps_cpu) < 0.05


def full_trainer(name, **kw):
    w = workloads()[name]
    lay = w.layout
    maps = synth.material(w.seed, lay.W, lay.H) if lay.T == 4 else [synth.rgb_texture(w.seed, lay.W, lay.H)]
    tgt = synth.target_from_maps(maps)
    z, p = synth.init_model(lay, w.seed, qat_bits=w.qat_bits)
    if w.dct_q:
        basis, zz = dct_tables(_orc())
        kw.update(dct={"C": lay.levels[0][2], "q": w.dct_q, "dc_step": 4}, dct_basis=basis, dct_zigzag=zz)
    tr = trainer(lay, z, p, tgt, max_pairs=w.mlp_pairs, max_batch=w.mlp_batch, seed=w.seed, qat_bits=w.qat_bits,
                 qat_grid=synth.qat_grid() if w.qat_bits else None, **kw)
    return w, lay, tr, z, p, tgt


def _orc():
    return oracle()


def live_dct(orc, w, lay, tr, z, p, tgt):
    """the workload's --dct-q level switched live as the reference's DCT switch does it (main.cpp:4099-4120):
    scale codes from the decoder sensitivity probe (the device's, checked against the oracle's), the host
    snap of the shadow, set_dct; then one rate-pass latent step with lr 0 and the device snap, all exact
    against the oracle at the full size"""
    H = HostDct(orc, lay, w.dct_q, deadzone=0, lam=0.5, lo16=4, rate="both")
    n0 = lay.levels[0][0] * lay.levels[0][1] * lay.levels[0][2]
    zd, _ = tr.download_model()
    assert np.array_equal(zd[:n0], np.clip(z[:n0], -1, 1))
    code_d, _ = tr.dct_probe()
    H.probe(lay, p, tr.download_zq())
    differ = int((code_d != H.code).sum())
    say(f"{w.name}: device probe codes differing from the oracle's: {differ} of {H.n}")
    assert differ <= max(2, H.n // 100) and np.all(np.abs(code_d.astype(int) - H.code.astype(int)) <= 1)
    H.code[:] = code_d
    zs, zq, bits, cnt = H.snap(zd)
    tr.set_dct(H.desc(), H.code, H.sym, H.steps)
    sym_d, c_d = tr.download_dct()
    assert np.array_equal(sym_d, H.sym) and np.array_equal(c_d, H.code)
    assert np.array_equal(tr.download_zq()[:n0], zq)
    K = w.lat_pairs
    tr.lat_step(1, w.lat_sigma, 0.0, K)               # the rate pass of every pair; lr 0 leaves the shadow
    zd2, _ = tr.download_model()
    assert np.array_equal(zd2, zd)
    bits_d, dbits_d, nt_d, nz_d, hits_d, evals_d = tr.download_dct_rate()
    zdec = tr.download_zq()
    g_o, _, dbits_o, hits_o = orc.lat_grad(lay, p, zdec, zd2, tgt, w.seed, 0, w.lat_sigma, K, 3, dct=H.d,
                                           rate_scale=float(H.rate_scale))
    say(f"{w.name}: rate pass bit differences nonzero on {hits_d} of {H.n * K} (block, channel, pair)")
    assert np.array_equal(dbits_d, dbits_o) and hits_d == hits_o and evals_d == H.n * K
    g = tr.debug_last_zgrad()
    assert np.abs(g - g_o).max() < 1e-3 * np.sqrt((g_o.astype(np.float64) ** 2).mean())
    zs2, zq2, bits2, cnt2 = H.snap(zd2)
    sym_d, _ = tr.download_dct()
    assert np.array_equal(sym_d, H.sym) and np.array_equal(tr.download_zq()[:n0], zq2)
    assert np.array_equal(bits_d, bits2) and (nt_d, nz_d) == (cnt2[0], cnt2[1])
    say(f"{w.name}: snap of {H.n} blocks exact: {int(bits2.sum())} proxy bits/16, {nt_d} ACs truncated of {nz_d}")
    return H


@pytest.mark.parametrize("name", ["rgb256", "rgb512_two_level", "material512", "dct512", "material2048"])
def test_full_size_properties(orc, name):
    say("full size", name)
    w, lay, tr, z, p, tgt = full_trainer(name)
    if w.dct_q:
        live_dct(orc, w, lay, tr, z, p, tgt)
    zdec = tr.download_zq()                             # what every decode reads (the snapped plane with --dct-q)
    N, M = w.mlp_pairs, w.mlp_batch
    tr.mlp_step(1, w.mlp_sigma, 0.0, N, M)              # lr 0: Adam leaves every weight bit-identical
    assert np.array_equal(tr.download_model()[1], p)
    dl = tr.debug_last_dl()
    lp, lm = tr.debug_last_losses()
    idx = tr.debug_last_batch()
    assert np.array_equal(idx, orc.draw_batch(w.seed, 1, M, lay.W * lay.H))
    assert dl.size == N and np.isfinite(lp).all() and np.isfinite(lm).all()
    assert np.array_equal(dl, lp - lm) or np.abs(dl - (lp - lm)).max() <= 1e-15 * np.abs(lp).max()
    s = np.float64(np.float32(w.mlp_sigma))
    worst = 0.0
    for i in ((0, N // 2, N - 1) if M <= 65536 else (0, N - 1)):   # sampled pairs on the device's own minibatch
        eps = orc.gauss_fill(w.seed, 2, 1, i, 0, p.size).astype(np.float64)
        # w +- sigma eps as one rounding (sigma * eps is exact in double)
        wp = (p.astype(np.float64) + s * eps).astype(np.float32)
        wm = (p.astype(np.float64) - s * eps).astype(np.float32)
        worst = max(worst, rel(lp[i], orc.loss_subset(lay, wp, zdec, tgt, idx)), rel(lm[i], orc.loss_subset(lay, wm, zdec, tgt, idx)))
    say(f"{name}: sampled member losses within {worst:.2e} relative of the oracle")
    assert worst < 1e-5
    # the unperturbed pair of a central-difference step is the loss of w on the step's minibatch
    h = np.float32(w.fd_h)
    tr.mlp_step_fd(2, h, 0.0, M)
    l0, _ = tr.mlp_stats()
    idx_fd = tr.debug_last_batch()
    assert rel(l0, orc.loss_subset(lay, p, zdec, tgt, idx_fd)) < 1e-6
    dl_fd = tr.debug_last_dl()
    assert dl_fd.size == p.size and np.isfinite(dl_fd).all()
    # every weight's loss difference L(w_j + h) - L(w_j - h) (main.cpp:1890-1920) against the oracle on the device's own
    # minibatch, to 1e-3 of their RMS (the reference's own bar is 1e-2, main.cpp:3034); where the oracle would take
    # minutes (more than ~100 GFLOP), at weights sampled over every layer
    hh = (p + h).astype(np.float64) - (p - h).astype(np.float64)    # the steps as realized in float
    rms = np.sqrt((dl_fd ** 2).mean())
    if 2 * p.size * M * macs(lay) <= 60e9:
        dl_o, hh_o, l0_o = orc.mlp_fd_eval(lay, p, zdec, tgt, h, idx_fd)
        assert np.array_equal(hh_o, hh) and rel(l0, l0_o) < 1e-6
        js = np.arange(p.size)
    else:
        js = np.unique(np.linspace(0, p.size - 1, 12 if M > 65536 else 24).astype(int))
        dl_o = np.zeros(p.size)
        for j in js:
            wpj, wmj = p.copy(), p.copy()
            wpj[j], wmj[j] = p[j] + h, p[j] - h
            dl_o[j] = orc.loss_subset(lay, wpj, zdec, tgt, idx_fd) - orc.loss_subset(lay, wmj, zdec, tgt, idx_fd)
    err = np.abs(dl_fd[js] - dl_o[js]).max() / rms
    say(f"{name}: central differences of {js.size} of {p.size} weights within {err:.2e} of their RMS ({rms:.3e})")
    assert err < 1e-3
    # Adam on the central-difference gradient, after the reset of the switch (main.cpp:4075-4084), bit for bit
    tr.reset_mlp_adam()
    tr.mlp_step_fd(2, h, w.mlp_lr, M)
    assert np.array_equal(tr.debug_last_dl(), dl_fd)
    pf, m0, v0 = p.copy(), np.zeros_like(p), np.zeros_like(p)
    orc.adam(pf, orc.fd_grad(dl_fd, hh), m0, v0, w.mlp_lr, 1)
    assert np.array_equal(tr.download_model()[1], pf)
    tr.mlp_step(3, w.mlp_sigma, w.mlp_lr, N, M)
    assert np.isfinite(tr.download_model()[1]).all()
    tr.lat_step(1, w.lat_sigma, w.lat_lr, w.lat_pairs)
    g = tr.debug_last_zgrad()
    assert np.isfinite(g).all()
    n0 = lay.levels[0][0] * lay.levels[0][1] * lay.levels[0][2]
    if w.qat_bits:
        assert not g[:n0].any() and g[n0:].any()
        tr.qat_search()
        zq = tr.download_model()[0][:n0].reshape(-1, lay.levels[0][2])
        grid = synth.qat_grid()
        for c, b in enumerate(w.qat_bits):
            assert np.array_equal(synth.qat_snap(zq[:, c], b, grid), zq[:, c])
    else:
        assert g[:n0].any()
    img = tr.decode_full()
    assert np.isfinite(img).all() and img.min() >= 0 and img.max() <= 1


def macs(lay) -> int:
    w = [lay.nin] + list(lay.hidden) + [lay.nout]
    return sum(w[i] * w[i + 1] for i in range(len(w) - 1))


def mse_psnr(orc, img, tgt, lay):
    """the reference's printed figure: mse_of (both images rounded to 8 bits, main.cpp:1764-1788), 10 log10(255^2 / mse)"""
    tex, weighted = np.zeros(4), np.zeros(1)
    cw = [float(x) for x in (lay.weights or [1.0] * lay.T)]
    wv = np.array(cw, np.float32)
    orc._mse_of(img.ctypes.data, tgt.ctypes.data, lay.W, lay.H, lay.nout, wv.ctypes.data, float(np.float32(wv.sum())), 0, 0,
                tex.ctypes.data, weighted.ctypes.data)
    mse = float(weighted[0])                        # in 8-bit units
    return mse, 10 * np.log10(255.0 ** 2 / mse)


@pytest.mark.skipif(not have_reference(fast=True), reason="the reference's CPU loop is built only where the reference tree is")
def test_rgb256_fixed_seed_psnr(orc):
    """rgb256 (the CPU-reference plumbing run) trained for its full 200 iterations at its fixed seed on the
    device and by the reference's own CPU training loop (main.cpp compiled with its -O3 -ffast-math flags,
    MlpTrainer / LatentTrainer in main.cpp:4121-4148's order, --rng hash), from the same initial model: the
    final PSNRs must agree within 0.05 dB (the reference's own cross-backend check, README.md:964-970)."""
    w, lay, tr, z, p, tgt = full_trainer("rgb256")
    ref = reference(fast=True)
    cfg = OrTrainCfg()
    cfg.seed, cfg.mlp_pairs, cfg.mlp_batch, cfg.mlp_sigma, cfg.mlp_lr = w.seed, w.mlp_pairs, w.mlp_batch, w.mlp_sigma, w.mlp_lr
    cfg.lat_pairs, cfg.lat_sigma, cfg.lat_lr, cfg.fd_from, cfg.fd_h = w.lat_pairs, w.lat_sigma, w.lat_lr, w.iters + 1, w.fd_h
    mc = model_of(lay)
    h = ref.lib.ref_train_create(C.byref(mc), C.byref(cfg), z.ctypes.data, p.ctypes.data, tgt.ctypes.data)
    t0 = time.time()
    try:
        for it in range(1, w.iters + 1):
            ref.lib.ref_train_iter(h, it, w.iters)
            if it % 50 == 0:
                say(f"rgb256 reference CPU loop: iteration {it} ({time.time() - t0:.1f} s)")
        zr, pr = np.empty_like(z), np.empty_like(p)
        ref.lib.ref_train_get(h, zr.ctypes.data, pr.ctypes.data)
    finally:
        ref.lib.ref_train_destroy(h)
    t1 = time.time()
    for it in range(1, w.iters + 1):
        tr.mlp_step(it, w.mlp_sigma, w.mlp_lr, w.mlp_pairs, w.mlp_batch)
        tr.lat_step(it, w.lat_sigma, w.lat_lr, w.lat_pairs)
    img = tr.decode_full()
    t2 = time.time()
    mse_0, ps_0 = mse_psnr(orc, orc.decode_full(lay, p, z), tgt, lay)
    mse_c, ps_c = mse_psnr(orc, orc.decode_full(lay, pr, zr), tgt, lay)
    mse_g, ps_g = mse_psnr(orc, img, tgt, lay)
    say(f"rgb256 {w.iters} iterations, seed {w.seed}: start psnr {ps_0:.3f} dB; reference CPU loop mse {mse_c:.3f} psnr "
        f"{ps_c:.3f} dB ({t1 - t0:.1f} s); device mse {mse_g:.3f} psnr {ps_g:.3f} dB ({t2 - t1:.2f} s); "
        f"delta {ps_g - ps_c:+.4f} dB")
    assert ps_c > ps_0 + 1.0                            # training moved
    assert abs(ps_g - ps_c) <= 0.05


@pytest.mark.skipif(not have_reference(fast=True), reason="the reference's CPU loop is built only where the reference tree is")
def test_material512_fixed_seed_psnr(orc):
    """material512 (the headline workload: four 512x512 maps, --qat 2,2 on level 0, population 8192 on 4096-pixel
    minibatches) trained for 20 iterations at its fixed seed on the device and by the reference's own CPU training
    loop (main.cpp's MlpTrainer / LatentTrainer / qat_search in main.cpp:4121-4148's order, -O3 -ffast-math,
    --rng hash), from the same initial model: the final PSNRs must agree within 0.05 dB (README.md:964-970)."""
    iters = 20
    w, lay, tr, z, p, tgt = full_trainer("material512")
    ref = reference(fast=True)
    cfg = OrTrainCfg()
    cfg.seed, cfg.mlp_pairs, cfg.mlp_batch, cfg.mlp_sigma, cfg.mlp_lr = w.seed, w.mlp_pairs, w.mlp_batch, w.mlp_sigma, w.mlp_lr
    cfg.lat_pairs, cfg.lat_sigma, cfg.lat_lr, cfg.fd_from, cfg.fd_h = w.lat_pairs, w.lat_sigma, w.lat_lr, iters + 1, w.fd_h
    cfg.qat = max(w.qat_bits)
    for c, b in enumerate(w.qat_bits):
        cfg.qat_ch[c] = b
    mc = model_of(lay)
    h = ref.lib.ref_train_create(C.byref(mc), C.byref(cfg), z.ctypes.data, p.ctypes.data, tgt.ctypes.data)
    t0 = time.time()
    try:
        for it in range(1, iters + 1):
            ref.lib.ref_train_iter(h, it, iters)
            if it % 5 == 0:
                say(f"material512 reference CPU loop: iteration {it} ({time.time() - t0:.1f} s)")
        zr, pr = np.empty_like(z), np.empty_like(p)
        ref.lib.ref_train_get(h, zr.ctypes.data, pr.ctypes.data)
    finally:
        ref.lib.ref_train_destroy(h)
    t1 = time.time()
    for it in range(1, iters + 1):
        tr.mlp_step(it, w.mlp_sigma, w.mlp_lr, w.mlp_pairs, w.mlp_batch)
        tr.lat_step(it, w.lat_sigma, w.lat_lr, w.lat_pairs)
        tr.qat_search()
    img = tr.decode_full()
    t2 = time.time()
    mse_0, ps_0 = mse_psnr(orc, orc.decode_full(lay, p, z), tgt, lay)
    mse_c, ps_c = mse_psnr(orc, orc.decode_full(lay, pr, zr), tgt, lay)
    mse_g, ps_g = mse_psnr(orc, img, tgt, lay)
    say(f"material512 {iters} iterations, seed {w.seed}: start psnr {ps_0:.3f} dB; reference CPU loop mse {mse_c:.3f} psnr "
        f"{ps_c:.3f} dB ({t1 - t0:.1f} s); device mse {mse_g:.3f} psnr {ps_g:.3f} dB ({t2 - t1:.2f} s); "
        f"delta {ps_g - ps_c:+.4f} dB")
    assert ps_c > ps_0 + 0.5                            # training moved
    assert abs(ps_g - ps_c) <= 0.05


def _reference_loop(w, lay, z, p, tgt, iters, dct=None):
    """the reference's own CPU training loop (libntc_ref_fast.so, --rng hash) for `iters` iterations from (z, p):
    the final shadow and weights"""
    ref = reference(fast=True)
    cfg = OrTrainCfg()
    cfg.seed, cfg.mlp_pairs, cfg.mlp_batch, cfg.mlp_sigma, cfg.mlp_lr = w.seed, w.mlp_pairs, w.mlp_batch, w.mlp_sigma, w.mlp_lr
    cfg.lat_pairs, cfg.lat_sigma, cfg.lat_lr, cfg.fd_from, cfg.fd_h = w.lat_pairs, w.lat_sigma, w.lat_lr, iters + 1, w.fd_h
    cfg.qat = max(w.qat_bits) if w.qat_bits else 0
    for c, b in enumerate(w.qat_bits or []):
        cfg.qat_ch[c] = b
    mc = model_of(lay)
    if dct is None:
        h = ref.lib.ref_train_create(C.byref(mc), C.byref(cfg), z.ctypes.data, p.ctypes.data, tgt.ctypes.data)
    else:
        h = ref.lib.ref_train_create_dct(C.byref(mc), C.byref(cfg), z.ctypes.data, p.ctypes.data, tgt.ctypes.data, C.byref(dct.d),
                                         C.c_float(0.5), 1, 1)
    t0 = time.time()
    try:
        for it in range(1, iters + 1):
            ref.lib.ref_train_iter(h, it, iters)
        zr, pr = np.empty_like(z), np.empty_like(p)
        ref.lib.ref_train_get(h, zr.ctypes.data, pr.ctypes.data)
    finally:
        ref.lib.ref_train_destroy(h)
    return zr, pr, time.time() - t0


@pytest.mark.skipif(not have_reference(fast=True), reason="the reference's CPU loop is built only where the reference tree is")
def test_rgb512_two_level_fixed_seed_psnr(orc):
    """rgb512_two_level (two bilinear levels, 32-wide MLP, population 1024 on 64K-pixel minibatches) trained for 10
    iterations at its fixed seed on the device and by the reference's own CPU loop: final PSNRs within 0.05 dB."""
    iters = 10
    w, lay, tr, z, p, tgt = full_trainer("rgb512_two_level")
    zr, pr, el = _reference_loop(w, lay, z, p, tgt, iters)
    for it in range(1, iters + 1):
        tr.mlp_step(it, w.mlp_sigma, w.mlp_lr, w.mlp_pairs, w.mlp_batch)
        tr.lat_step(it, w.lat_sigma, w.lat_lr, w.lat_pairs)
    img = tr.decode_full()
    _, ps_0 = mse_psnr(orc, orc.decode_full(lay, p, z), tgt, lay)
    mse_c, ps_c = mse_psnr(orc, orc.decode_full(lay, pr, zr), tgt, lay)
    mse_g, ps_g = mse_psnr(orc, img, tgt, lay)
    say(f"rgb512_two_level {iters} iterations, seed {w.seed}: start psnr {ps_0:.3f} dB; reference CPU loop mse {mse_c:.3f} "
        f"psnr {ps_c:.3f} dB ({el:.1f} s); device mse {mse_g:.3f} psnr {ps_g:.3f} dB; delta {ps_g - ps_c:+.4f} dB")
    assert ps_c > ps_0 + 0.5
    assert abs(ps_g - ps_c) <= 0.05


@pytest.mark.skipif(not have_reference(fast=True), reason="the reference's CPU loop is built only where the reference tree is")
def test_dct512_fixed_seed_psnr(orc):
    """dct512 (a --dct-q 50 plane as level 0 with the rate proxy in the objective, scale codes from the device's
    decoder-sensitivity probe) trained for 20 iterations at its fixed seed on the device and by the reference's own
    CPU loop with the same DCT state (codes, steps, --dct-lambda 0.5 with both parts, the shadow pulled toward the
    plane by --dct-shadow-pull 0.01 after every latent step): the final PSNRs of the decoded (snapped) models within
    0.05 dB."""
    iters = 20
    w, lay, tr, z, p, tgt = full_trainer("dct512")
    H = HostDct(orc, lay, w.dct_q, deadzone=0, lam=0.5, lo16=4, rate="both")
    code_d, _ = tr.dct_probe()
    H.code[:] = code_d
    zd, _ = tr.download_model()                       # the shadow as the trainer holds it (level 0 clamped)
    H.snap(zd)
    tr.set_dct(H.desc(), H.code, H.sym, H.steps)
    zr, pr, el = _reference_loop(w, lay, zd, p, tgt, iters, dct=H)   # with the default --dct-shadow-pull 0.01
    n0 = lay.levels[0][0] * lay.levels[0][1] * lay.levels[0][2]
    for it in range(1, iters + 1):
        tr.mlp_step(it, w.mlp_sigma, w.mlp_lr, w.mlp_pairs, w.mlp_batch)
        tr.lat_step(it, w.lat_sigma, w.lat_lr, w.lat_pairs)
        tr.shadow_pull(0, n0, w.shadow_pull)       # main.cpp:4136
    img = tr.decode_full()
    _, zq_r, _, _ = H.snap(zr)                        # the reference's final plane, snapped with the same codes
    _, zq_0, _, _ = H.snap(zd)
    _, ps_0 = mse_psnr(orc, orc.decode_full(lay, p, np.concatenate([zq_0, zd[n0:]])), tgt, lay)
    mse_c, ps_c = mse_psnr(orc, orc.decode_full(lay, pr, np.concatenate([zq_r, zr[n0:]])), tgt, lay)
    mse_g, ps_g = mse_psnr(orc, img, tgt, lay)
    say(f"dct512 {iters} iterations, seed {w.seed}: start psnr {ps_0:.3f} dB; reference CPU loop mse {mse_c:.3f} psnr "
        f"{ps_c:.3f} dB ({el:.1f} s); device mse {mse_g:.3f} psnr {ps_g:.3f} dB; delta {ps_g - ps_c:+.4f} dB")
    assert ps_c > ps_0 + 0.5
    assert abs(ps_g - ps_c) <= 0.05


def test_material512_selectors_full_size(orc):
    """One selector search (--qat 2,2, qat_search main.cpp:2088-2139) at material512's full size (262144 texels x
    2 channels, 12 outputs), after a few training iterations on the device, against the oracle's search of the
    same model. Every texel channel whose choice differs is counted and printed; at each one the reference's
    cell losses (loss_subset of the one pixel, the double sum of float terms) of the two choices must agree to
    a rounding tie (the reference's own check accepts ties, main.cpp:3143-3144)."""
    w, lay, tr, z, p, tgt = full_trainer("material512")
    for it in range(1, 6):
        tr.mlp_step(it, w.mlp_sigma, w.mlp_lr, w.mlp_pairs, w.mlp_batch)
        tr.lat_step(it, w.lat_sigma, w.lat_lr, w.lat_pairs)
        tr.qat_search()
    zd, pd = tr.download_model()
    tr.qat_search()
    z_dev = tr.download_model()[0]
    z_or = zd.copy()
    grid = synth.qat_grid()
    orc.qat_search(lay, pd, z_or, tgt, w.qat_bits, grid)
    W0, H0, C0, _ = lay.levels[0]
    n0 = W0 * H0 * C0
    a, b, before = z_dev[:n0].reshape(-1, C0), z_or[:n0].reshape(-1, C0), zd[:n0].reshape(-1, C0)
    diff = np.nonzero((a != b).any(axis=1))[0]
    changed = int((b != before).any(axis=1).sum())
    worst = 0.0
    for t in diff:
        c = int(np.nonzero(a[t] != b[t])[0][0])            # the first channel whose choice differs
        losses = []
        for v in (a[t, c], b[t, c]):
            zz = zd.copy()
            zz[t * C0:(t + 1) * C0] = np.concatenate([b[t, :c], [v], before[t, c + 1:]])
            losses.append(orc.loss_subset(lay, pd, zz, tgt, np.array([t], np.int32)))
        gap = abs(losses[0] - losses[1]) / max(abs(losses[1]), 1e-30)
        worst = max(worst, gap)
    say(f"material512 selector search: {diff.size} of {W0 * H0} texels ({2 * W0 * H0} channel choices) differ from the "
        f"oracle's; the oracle changed {changed} texels; largest relative cell-loss gap at a difference {worst:.2e}")
    assert diff.size <= max(2, W0 * H0 // 1000)
    assert worst < 1e-5
