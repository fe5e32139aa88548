"""HIP kernels through the C ABI against the oracle, on identical seeded inputs.

Bars: noise, minibatch indices, --qes indices and values, DCT symbols / codes / planes / bit counts
and Adam / ES-update arithmetic are bit-exact; per-member ES losses within 1e-5 relative (the
task's bar); decoded values within 2e-6 absolute (the device's expf against the host C
library's is the only difference on this path); latent gradients within 1e-3 of their RMS (the
reference's own --cuda-check bar, main.cpp:3088); qat selectors equal except on texels whose two
candidates have cell losses equal to 1e-6 relative (main.cpp:3143-3144)."""
import numpy as np
import pytest

from neural_block_textures_amd import synth
from tests.gpu_common import LAYOUTS, data, rel, say, trainer

pytestmark = pytest.mark.gpu
NAMES = list(LAYOUTS)


def test_noise_factors_exhaustive(orc):
    """Every one of the 2^24 values of each Box-Muller factor on the device equals the host's."""
    lay = LAYOUTS["rgb_16x2"]
    z, p, tgt = data(lay, 1)
    tr = trainer(lay, z, p, tgt)
    n = 1 << 24
    rad_d, cos_d = tr.debug_noise_factors(0, n)
    rad_h, cos_h = np.empty(n, np.float32), np.empty(n, np.float32)
    orc._gauss_factors(0, n, rad_h.ctypes.data, cos_h.ctypes.data)
    assert np.array_equal(rad_d.view(np.uint32), rad_h.view(np.uint32))
    assert np.array_equal(cos_d.view(np.uint32), cos_h.view(np.uint32))
    for stream, step, pair in [(1, 0, 0), (2, 7, 4095), (3, 123456, 0), (1, 2**20, 3)]:
        say("gauss stream", stream, step, pair)
        g = tr.debug_gauss(stream, step, pair, 0, 1 << 20)
        want = orc.gauss_fill(5, stream, step, pair, 0, 1 << 20)
        assert np.array_equal(g.view(np.uint32), want.view(np.uint32))
    g = tr.debug_gauss(2, 1, 1, 2**40 - 100, 200)
    assert np.array_equal(g.view(np.uint32), orc.gauss_fill(5, 2, 1, 1, 2**40 - 100, 200).view(np.uint32))


@pytest.mark.parametrize("name", NAMES)
def test_decode(orc, name):
    lay = LAYOUTS[name]
    say("decode", name)
    z, p, tgt = data(lay, 2)
    tr = trainer(lay, z, p, tgt)
    img = tr.decode_full()
    want = orc.decode_full(lay, p, z)
    if lay.clamp_out:
        assert np.array_equal(img, want)
    else:
        assert np.abs(img - want).max() < 2e-6
        assert (img == want).mean() > 0.95
    z2 = (z * np.float32(0.5)).astype(np.float32)   # a host-supplied latent
    assert np.abs(tr.decode_full(z2) - orc.decode_full(lay, p, z2)).max() < 2e-6


@pytest.mark.parametrize("name", NAMES)
def test_mlp_es_step(orc, name):
    lay = LAYOUTS[name]
    say("mlp es", name)
    z, p, tgt = data(lay, 3)
    N, M, seed, it, sigma, lr = 200, 1500, 5, 7, 0.02, 0.005
    tr = trainer(lay, z, p, tgt, max_pairs=N, max_batch=M, seed=seed)
    tr.mlp_step(it, sigma, lr, N, M)
    idx = orc.draw_batch(seed, it, M, lay.W * lay.H)
    assert np.array_equal(tr.debug_last_batch(), idx)
    lp, lm = tr.debug_last_losses()
    dl_o, _, lp_o, lm_o = orc.mlp_es_eval(lay, p, z, tgt, seed, it, sigma, N, idx)
    assert rel(lp, lp_o).max() < 1e-5 and rel(lm, lm_o).max() < 1e-5
    dl = tr.debug_last_dl()
    assert np.abs(dl - dl_o).max() / np.sqrt((dl_o ** 2).mean()) < 1e-3
    # the update direction from the device's own pair differences: the device adds the pairs in
    # chains of 32 combined in a fixed order, the reference in one chain; Adam on it is bit-exact
    g_o = orc.mlp_es_grad(p.size, N, seed, it, sigma, dl)
    g = tr.debug_last_wgrad()
    assert np.abs(g - g_o).max() <= 1e-5 * np.abs(g_o).max()
    if N <= 32:
        assert np.array_equal(g, g_o)                   # one chain: the reference's order exactly
    pw, m, v = p.copy(), np.zeros_like(p), np.zeros_like(p)
    orc.adam(pw, g, m, v, lr, 1)
    _, p_dev = tr.download_model()
    assert np.array_equal(p_dev, pw)
    loss, dstd = tr.mlp_stats()
    assert abs(loss - 0.5 * (lp + lm).mean()) < 1e-12 and dstd > 0


@pytest.mark.parametrize("name", ["rgb_16x2", "material", "dct_plane", "two_level", "dct_17", "chief1_36", "runtime", "jit_widths",
                                  "material_valu"])
def test_mlp_es_small_batches(orc, name):
    """minibatches of less than one 16-slot tile, one slot past a tile and a few tiles, and one or a few pairs, on
    one trainer in a row (each call sizes its own chunks): member losses to the bar, the update one chain exactly, and
    Adam on it bit-exact"""
    lay = LAYOUTS[name]
    say("mlp es small", name)
    z, p, tgt = data(lay, 6)
    seed, sigma, lr = 11, 0.02, 0.005
    tr = trainer(lay, z, p, tgt, max_pairs=8, max_batch=64, seed=seed)
    pw, m, v = p.copy(), np.zeros_like(p), np.zeros_like(p)
    for t, (it, N, M) in enumerate([(1, 1, 1), (2, 3, 13), (3, 5, 17), (4, 2, 33), (5, 8, 64)], start=1):
        tr.mlp_step(it, sigma, lr, N, M)
        idx = orc.draw_batch(seed, it, M, lay.W * lay.H)
        assert np.array_equal(tr.debug_last_batch(), idx)
        lp, lm = tr.debug_last_losses()
        dl_o, _, lp_o, lm_o = orc.mlp_es_eval(lay, pw, z, tgt, seed, it, sigma, N, idx)
        assert lp.size == N and rel(lp, lp_o).max() < 1e-5 and rel(lm, lm_o).max() < 1e-5, (N, M)
        g = orc.mlp_es_grad(p.size, N, seed, it, sigma, tr.debug_last_dl())
        assert np.array_equal(tr.debug_last_wgrad(), g), (N, M)
        orc.adam(pw, g, m, v, lr, t)
        assert np.array_equal(tr.download_model()[1], pw), (N, M)


@pytest.mark.parametrize("name", ["rgb_16x2", "material", "runtime", "chief1_36", "dct_17", "dct_11", "material_valu", "jit_valu_7",
                                  "jit_mfma_28", "jit_own_13", "jit_widths"])
def test_mlp_es_two_steps_and_fd(orc, name):
    lay = LAYOUTS[name]
    say("mlp es+fd", name)
    z, p, tgt = data(lay, 4)
    N, M, seed = 8, 700, 9
    tr = trainer(lay, z, p, tgt, max_pairs=N, max_batch=M, seed=seed)
    pw, m, v = p.copy(), np.zeros_like(p), np.zeros_like(p)
    for t, it in [(1, 3), (2, 4)]:
        tr.mlp_step(it, 0.02, 0.005, N, M)
        g = orc.mlp_es_grad(p.size, N, seed, it, 0.02, tr.debug_last_dl())
        assert np.array_equal(tr.debug_last_wgrad(), g)   # N <= 32: a single chain, the reference's order
        orc.adam(pw, g, m, v, 0.005, t)
    _, p_dev = tr.download_model()
    assert np.array_equal(p_dev, pw)
    # central differences after an Adam reset, from the weights the ES steps left
    tr.reset_mlp_adam()
    h = np.float32(1e-3)
    tr.mlp_step_fd(5, h, 0.005, M)
    idx = orc.draw_batch(seed, 5, M, lay.W * lay.H)
    dl_o, hh, l0 = orc.mlp_fd_eval(lay, pw, z, tgt, h, idx)
    dl = tr.debug_last_dl()
    lp, lm = tr.debug_last_losses()
    assert dl.size == p.size
    assert np.abs(dl - dl_o).max() / np.sqrt((dl_o ** 2).mean()) < 1e-3
    assert rel(lp[0], l0) < 1e-3   # l(w_0 + h) against l(w): same batch, one weight moved by h
    loss, _ = tr.mlp_stats()
    assert rel(loss, l0) < 1e-5
    pf, m0, v0 = pw.copy(), np.zeros_like(p), np.zeros_like(p)
    orc.adam(pf, orc.fd_grad(dl, hh), m0, v0, 0.005, 1)
    assert np.array_equal(tr.download_model()[1], pf)


@pytest.mark.parametrize("name", NAMES)
def test_latent_gather_exact(orc, name):
    """the footprint gather sums every texel's pixel rectangle in raster order, as the reference's scatter: the
    latent gradient is the oracle's scatter of the device's own per-pixel differences, bit for bit (4 pairs per
    block: 1 and 3 pairs, and 6 in two rounds)"""
    lay = LAYOUTS[name]
    say("latent gather", name)
    z, p, tgt = data(lay, 5)
    seed, sigma = 7, np.float32(0.05)
    mask = (1 << len(lay.levels)) - 1
    for K in (1, 3, 6):
        tr = trainer(lay, z, p, tgt, seed=seed)
        tr.lat_step(1, sigma, 0.02, K)
        dpix = tr.debug_last_dpix()
        assert dpix.shape == (K, lay.W * lay.H)
        eps = np.concatenate([orc.gauss_fill(seed, 1, 0, k, 0, lay.nz) for k in range(K)])
        assert np.array_equal(tr.debug_last_zgrad(), orc.lat_scatter(lay, eps, dpix, K, mask, sigma))


@pytest.mark.parametrize("name", NAMES)
def test_latent_step(orc, name):
    lay = LAYOUTS[name]
    say("latent", name)
    z, p, tgt = data(lay, 5)
    K, seed, sigma, lr = 3, 7, 0.05, 0.02
    tr = trainer(lay, z, p, tgt, seed=seed)
    tr.lat_step(1, sigma, lr, K)
    mask = (1 << len(lay.levels)) - 1
    g_o, _, _, _ = orc.lat_grad(lay, p, z, z, tgt, seed, 0, sigma, K, mask)
    g = tr.debug_last_zgrad()
    rms = np.sqrt((g_o.astype(np.float64) ** 2).mean())
    assert np.abs(g - g_o).max() < 1e-3 * rms
    zz, m, v = z.copy(), np.zeros_like(z), np.zeros_like(z)
    orc.adam(zz, g, m, v, lr, 1)
    assert np.array_equal(tr.download_model()[0], zz)
    # the second step keys its noise with step 1
    tr.lat_step(2, sigma, lr, K)
    g2_o, _, _, _ = orc.lat_grad(lay, p, zz, zz, tgt, seed, 1, sigma, K, mask)
    assert np.abs(tr.debug_last_zgrad() - g2_o).max() < 1e-3 * np.sqrt((g2_o.astype(np.float64) ** 2).mean())


QAT = {"material": [2, 3], "material_clamp": [2, 3], "dct_plane": [1], "runtime": [2, 1, 3], "chief1_36": [2], "mat_qat_36": [2, 2], "image3_27": [4],
       "material_valu": [2, 3], "chief1_36_valu": [2], "mat_qat1x4_36": [2], "jit_mfma_28": [2, 1], "jit_widths": [2, 1, 3]}


@pytest.mark.parametrize("name", list(QAT))
def test_qat_search_and_frozen_level(orc, name):
    lay = LAYOUTS[name]
    bits = QAT[name]
    say("qat", name)
    grid = synth.qat_grid()
    z, p, tgt = data(lay, 6)
    n0 = lay.levels[0][0] * lay.levels[0][1] * lay.levels[0][2]
    C0 = lay.levels[0][2]
    lv0 = z[:n0].reshape(-1, C0)
    for c in range(C0):
        lv0[:, c] = synth.qat_snap(lv0[:, c], bits[c], grid)
    z[:n0] = lv0.reshape(-1)
    tr = trainer(lay, z, p, tgt, qat_bits=bits, qat_grid=grid)
    # latent step with level 0 frozen: its gradient is exactly zero
    tr.lat_step(1, 0.05, 0.0, 2)
    g = tr.debug_last_zgrad()
    assert not g[:n0].any()
    mask = ((1 << len(lay.levels)) - 1) & ~1
    g_o, dpix_o, _, _ = orc.lat_grad(lay, p, z, z, tgt, 5, 0, 0.05, 2, mask, want_dpix=True)
    assert np.abs(g - g_o).max() < 1e-3 * np.sqrt((g_o.astype(np.float64) ** 2).mean())
    # the per-pixel differences with level 0 outside the perturbation mask (its texels taken unperturbed)
    dpix = tr.debug_last_dpix()
    assert np.abs(dpix.ravel() - dpix_o).max() < 1e-3 * np.sqrt((dpix_o.astype(np.float64) ** 2).mean())
    tr.qat_search()
    zg = tr.download_model()[0]
    zc = z.copy()
    orc.qat_search(lay, p, zc, tgt, bits, grid)
    assert np.array_equal(zg[n0:], z[n0:])            # only level 0 moves
    assert not np.array_equal(zc[:n0], z[:n0])        # the search did something
    diff = np.nonzero((zg[:n0] != zc[:n0]).reshape(-1, C0).any(1))[0]
    say("qat differing texels", diff.size, "of", n0 // C0)
    assert diff.size <= max(2, n0 // C0 // 100)
    if diff.size:   # each must be a near tie: equal cell losses to 1e-6 on the oracle
        ec = orc.decode_err(lay, p, zc, tgt)
        eg = orc.decode_err(lay, p, zg, tgt)
        W0, H0 = lay.levels[0][0], lay.levels[0][1]
        for t in diff:
            tx, ty = t % W0, t // W0
            xs = [px for px in range(lay.W) if min(W0 - 1, int(np.floor((px + 0.5) / lay.W * W0))) == tx]
            ys = [py for py in range(lay.H) if min(H0 - 1, int(np.floor((py + 0.5) / lay.H * H0))) == ty]
            cc = sum(float(ec[y * lay.W + x]) for y in ys for x in xs)
            cg = sum(float(eg[y * lay.W + x]) for y in ys for x in xs)
            assert abs(cc - cg) <= 1e-6 * max(cc, cg) + 1e-12
    # every level-0 value is on its channel's grid
    for c in range(C0):
        col = zg[:n0].reshape(-1, C0)[:, c]
        assert np.array_equal(synth.qat_snap(col, bits[c], grid), col)


@pytest.mark.parametrize("name,mfma", [("rgb_16x2", True), ("material", True), ("dct_17", True), ("jit_valu_7", False),
                                       ("material_valu", False)])
def test_matrix_core_choice(orc, name, mfma):
    """the populations run on the matrix cores from 40% useful multiply-adds on (17-wide hidden layers: 42-47%)"""
    lay = LAYOUTS[name]
    z, p, tgt = data(lay, 8)
    tr = trainer(lay, z, p, tgt)
    assert tr.on_matrix_cores("pop_eval") == mfma
    assert tr.on_matrix_cores("lat_pair") == mfma


@pytest.mark.parametrize("name,pair", [("material", True), ("dct_plane", True), ("two_level", True), ("rgb_16x2", True),
                                       ("large", False), ("dct_17", False), ("material_valu", False)])
def test_pair_population_kernel_choice(orc, name, pair):
    """ES steps share a pair's first layer on the fixed shapes with one or two 16-unit hidden tiles (k_pop_pair: the
    12-output material and the 3-output 32-wide ones; k_pop_pair_own: the pixel-per-lane 16-wide one); not the 64-wide
    one, a 17-wide one or the VALU kernels"""
    lay = LAYOUTS[name]
    z, p, tgt = data(lay, 8)
    tr = trainer(lay, z, p, tgt)
    assert tr.on_matrix_cores("pop_pair") == pair
    assert tr.on_matrix_cores("pop_pair_own") == (pair and name == "rgb_16x2")
    tr.close()


def test_pair_population_kernel_chunk_in_l2(orc):
    """the pair kernels read each chunk's first layer (H x chunk floats) from the L2: a step whose chunk would take more
    than 2 MiB evaluates on k_pop_mfma (2048 pairs of 65536 slots: one chunk, 8 MiB for 32 units), a step of the same
    model with fewer pairs (smaller chunks) on k_pop_pair"""
    lay = LAYOUTS["dct_plane"]
    z, p, tgt = data(lay, 8)
    for pairs, pair in ((2048, False), (64, True)):
        tr = trainer(lay, z, p, tgt, max_pairs=pairs, max_batch=65536)
        assert tr.on_matrix_cores("pop_pair") == pair, pairs
        tr.close()


@pytest.mark.parametrize("name", ["jit_valu_7", "jit_mfma_28", "jit_widths", "runtime"])
def test_specialised_shape_in_use(orc, name):
    """a shape the library does not list runs on kernels specialised for it at init (hidden layers of one width:
    FixedShape, of several: FixedShapeW), not the runtime-shaped ones, unless NTC_HIP_JIT=0 ("runtime")"""
    lay = LAYOUTS[name]
    z, p, tgt = data(lay, 8)
    tr = trainer(lay, z, p, tgt)
    say("banner", tr.banner())
    assert ("specialised at init" in tr.banner()) == (name != "runtime")
    if name == "jit_widths":
        assert "|20,12|" in tr.banner()
    assert tr.on_matrix_cores("pop_eval") == (name == "jit_mfma_28")


@pytest.mark.parametrize("name", ["rgb_16x2", "material", "large", "material_valu", "runtime"])
def test_nan_member_propagates(orc, name):
    """A diverged model (one NaN weight in the second hidden layer) behaves as in the reference, whose
    activation propagates a NaN (main.cpp:560): NaN member losses, a NaN update, a NaN decode and NaN
    per-pixel latent differences - on the matrix-core kernels (leak 0 and leak > 0) and on the VALU ones.
    With --clamp the reference's min(1, max(0, s + 0.5)) turns a NaN output into 0 (main.cpp:624): there
    every member's loss is the oracle's finite one and the decode is exactly the oracle's."""
    lay = LAYOUTS[name]
    say("nan", name)
    z, p, tgt = data(lay, 9)
    h = lay.hidden[0]
    p = p.copy()
    p[lay.nin * h + h + 3] = np.nan
    tr = trainer(lay, z, p, tgt, max_pairs=8, max_batch=512)
    tr.mlp_step(1, 0.02, 0.0, 8, 512)
    lp, lm = tr.debug_last_losses()
    l_o = orc.loss_subset(lay, p, z, tgt, tr.debug_last_batch())
    img = tr.decode_full()
    tr.lat_step(1, 0.05, 0.0, 2)
    dpix = tr.debug_last_dpix()
    if lay.clamp_out:
        assert np.isfinite(l_o) and rel(lp, l_o).max() < 1e-5 and rel(lm, l_o).max() < 1e-5
        assert np.array_equal(img, orc.decode_full(lay, p, z))
        assert not dpix.any()                       # every output is 0 for both members
    else:
        assert np.isnan(l_o) and np.isnan(lp).all() and np.isnan(lm).all()
        assert np.isnan(tr.debug_last_wgrad()).all()
        assert np.isnan(img).all() and np.isnan(dpix).all()
    tr.close()


@pytest.mark.parametrize("name,K", [("material", 512), ("rgb_16x2", 256)])
def test_latent_step_two_rounds(orc, name, K):
    """Enough pairs that ceil(W H / 512) K >= 2048: the latent pair kernel takes two 64-pixel rounds per wave
    (512-pixel blocks), the launch the full-size workloads use (models with at most 8 inputs). The per-pixel
    differences and the gradient against the oracle at the reference's bar (1e-3 of RMS, main.cpp:3088),
    the gather exactly as the oracle's scatter of the device's own differences, Adam bit for bit."""
    lay = LAYOUTS[name]
    assert lay.nin <= 8 and -(-lay.W * lay.H // 512) * K >= 2048
    say("latent two rounds", name, K)
    z, p, tgt = data(lay, 5)
    seed, sigma, lr = 7, np.float32(0.05), 0.02
    tr = trainer(lay, z, p, tgt, seed=seed)
    tr.lat_step(1, sigma, lr, K)
    mask = (1 << len(lay.levels)) - 1
    g_o, dpix_o, _, _ = orc.lat_grad(lay, p, z, z, tgt, seed, 0, sigma, K, mask, want_dpix=True)
    dpix = tr.debug_last_dpix()
    d_rms = np.sqrt((dpix_o.astype(np.float64) ** 2).mean())
    assert np.abs(dpix.ravel() - dpix_o).max() < 1e-3 * d_rms
    g = tr.debug_last_zgrad()
    assert np.abs(g - g_o).max() < 1e-3 * np.sqrt((g_o.astype(np.float64) ** 2).mean())
    eps = np.concatenate([orc.gauss_fill(seed, 1, 0, k, 0, lay.nz) for k in range(K)])
    assert np.array_equal(g, orc.lat_scatter(lay, eps, dpix, K, mask, sigma))
    zz, m, v = z.copy(), np.zeros_like(z), np.zeros_like(z)
    orc.adam(zz, g, m, v, lr, 1)
    assert np.array_equal(tr.download_model()[0], zz)
