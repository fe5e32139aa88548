"""Final PSNR of the device's training run against the reference's own CPU loop, at each benchmark workload's own
length and fixed seed (the reference's cross-backend check is a final PSNR, README.md:964-970; the loop is
main.cpp:4063-4239). The CPU side is a fixture: tests/golden/make_final_psnr.py ran ref_train_iter (the reference's
main.cpp compiled with its own flags) over the whole schedule in the build container and stored the PSNR at every
checkpoint and at the end. The device runs the same schedule through the Trainer interface, as main.cpp drives the
reference's backend (main.cpp:4075-4160): the ES steps, the switch to central differences with its Adam reset, the
selector search every iteration, the DCT switch with its probe and snap, the refits, the shadow pull, and the fp16
rounding of the final weights. Bar: |delta PSNR| <= 0.05 dB at the end."""
import os

import numpy as np
import pytest

from neural_block_textures_amd import dct_host, ntcb
from neural_block_textures_amd.trainer import DctDesc
from tests.golden.make_final_psnr import SCHEDULES, digest
from tests.gpu_common import say
from tests.test_gpu_training import full_trainer, mse_psnr

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixture(name):
    path = os.path.join(GOLDEN, f"final_psnr_{name}.npz")
    if not os.path.exists(path):
        pytest.skip(f"no reference run for {name} (tests/golden/make_final_psnr.py {name} writes it)")
    return np.load(path)


def dct_desc(w, lay, s):
    t16, scale = dct_host.lambda_weights(s["dct_lambda"], lay.W, lay.H, True, True)
    d = DctDesc()
    W0, H0, C0, _ = lay.levels[0]
    d.live, d.C, d.BW, d.BH, d.N, d.dc_step = 1, C0, W0 // 8, H0 // 8, 8, 4
    d.rate_es, d.rate_trunc, d.rate_scale = 1, 1, scale
    for k in range(16):
        d.lam_t16[k] = t16[k]
    d.lo_w16, d.deadzone = s["lo16"], 0
    steps = np.concatenate([dct_host.steps(q, 4).reshape(-1) for q in w.dct_q]).astype(np.int32)
    return d, steps, (W0 // 8) * (H0 // 8) * C0


@pytest.mark.parametrize("name", ["rgb256", "rgb512_two_level", "material512", "dct512", "material2048"])
def test_final_psnr_against_reference_loop(orc, name):
    fx = fixture(name)
    s = SCHEDULES[name]
    w, lay, tr, z, p, tgt = full_trainer(name)
    assert np.array_equal(digest(z, p, tgt), fx["digest"]), "the synthetic inputs differ from the reference run's"
    iters, fd_from, pairs = int(fx["iters"]), int(fx["fd_from"]), int(fx["pairs"])
    assert iters == s["iters"]
    n0 = lay.levels[0][0] * lay.levels[0][1] * lay.levels[0][2]
    live = False
    if w.dct_q:
        desc, steps, nblk = dct_desc(w, lay, s)
    checks = {int(c): (float(ps), float(m)) for c, ps, m in zip(fx["checkpoints"], fx["psnr"], fx["mse"])}
    worst = 0.0
    say(f"{name}: {iters} iterations on the device against the reference loop's fixture")
    for it in range(1, iters + 1):
        if w.dct_q:
            if not live and it == s["dct_start"]:                 # the DCT switch (main.cpp:4100-4109)
                code, _ = tr.dct_probe()                          # the probe of the clamped shadow, then the snap
                tr.set_dct(desc, code, np.zeros(nblk * 64, np.int16), steps)
                tr.snap_latent()
                live = True
            elif live and it % s["dct_refit"] == 0 and it < iters and it <= s["dct_refit_until"]:
                tr.dct_refit()                                    # main.cpp:4110-4120
        if it == fd_from:
            tr.reset_mlp_adam()                                   # main.cpp:4075-4084
        if it >= fd_from:
            tr.mlp_step_fd(it, np.float32(w.fd_h), w.mlp_lr, w.mlp_batch)
        else:
            tr.mlp_step(it, w.mlp_sigma, w.mlp_lr, pairs, w.mlp_batch)
        tr.lat_step(it, w.lat_sigma, w.lat_lr, w.lat_pairs)
        if live and s.get("shadow_pull"):
            tr.shadow_pull(0, n0, s["shadow_pull"])               # main.cpp:4136
        if w.qat_bits:
            tr.qat_search()
        if it in checks:
            _, ps = mse_psnr(orc, tr.decode_full(), tgt, lay)
            worst = max(worst, abs(ps - checks[it][0]))
            say(f"{name}: iteration {it}: device {ps:.4f} dB, reference {checks[it][0]:.4f} dB, delta {ps - checks[it][0]:+.4f}")
    if int(fx["fp16_end"]):                                       # --write-ntcb's rounding (main.cpp:4160)
        zf, pf = tr.download_model()
        tr.upload_model(zf, ntcb.round_fp16(pf))
    mse_g, ps_g = mse_psnr(orc, tr.decode_full(), tgt, lay)
    ps_c, mse_c = float(fx["final_psnr"]), float(fx["final_mse"])
    say(f"{name}: {iters} iterations, start {float(fx['start_psnr']):.4f} dB; reference CPU loop {ps_c:.4f} dB (mse {mse_c:.4f}, "
        f"{float(fx['cpu_seconds']):.0f} s on {int(fx['threads'])} threads); device {ps_g:.4f} dB (mse {mse_g:.4f}); "
        f"delta {ps_g - ps_c:+.4f} dB (largest at a checkpoint {worst:.4f})")
    tr.close()
    assert ps_c > float(fx["start_psnr"]) + 0.5                  # the run trained
    assert abs(ps_g - ps_c) <= 0.05
