"""Writes tests/golden/final_psnr_<workload>.npz: the final PSNR of the reference's own CPU training loop on a
benchmark workload, run for the workload's own length at its fixed seed.

The loop is ref_train_iter (oracle/ref_wrap.cpp: main.cpp's MlpTrainer / LatentTrainer / qat_search, the DCT switch
and refits, the shadow pull, in main.cpp:4063-4148's order, --rng hash), from oracle/_ref/libntc_ref_fast.so: the
reference's main.cpp compiled with its own -O3 -ffast-math flags for x86-64-v3. Run from the repository root in the
build container (the reference tree is read there only):

    make -C oracle ref && python tests/golden/make_final_psnr.py material512 [--state DIR] [--isa x86-64-v4]

Schedules (the reference's flags; C3-C5 of the workload descriptions):
  rgb256            200 iterations.
  rgb512_two_level  2000 iterations.
  material512       1050 iterations: 1000 ES iterations, --mlp-fd from iteration 1001 (main.cpp:3964-3965, the
                    Adam state reset at the switch, main.cpp:4075-4084), 50 central-difference iterations, the
                    selector search every iteration, then --write-ntcb's rounding of the weights to fp16
                    (main.cpp:2472-2481, 4160) before the final decode. The workload's own 8050 iterations take
                    about 7 hours of this container's 8 cores; 1000 ES iterations and the whole tail do not.
  dct512            4000 iterations: --dct-q 50, the switch at iteration 2000 (--dct-start 0.5, main.cpp:3804), a
                    refit every 500 iterations after it (main.cpp:3828-3830), --dct-lambda 0.5 with both parts,
                    --dct-lambda-lo 0.25, --dct-shadow-pull 0.01 after every latent step (main.cpp:4142-4146).
  material2048      10 iterations with 64 of its 8192 pairs, at the full image size.

Each file holds the inputs' SHA-256 (the synthetic generator's output, so a test can tell that it trains the same
model), the PSNR and mse of the decoded model (mse_of of main.cpp:1764-1788 on 8-bit values) at every checkpoint and
at the end, and the schedule. The loop's state is saved every few iterations under --state, so an interrupted run
resumes where it stopped. Data only.
"""
from __future__ import annotations

import argparse
import ctypes as C
import hashlib
import json
import math
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from neural_block_textures_amd import dct_host, synth  # noqa: E402
from neural_block_textures_amd.configs import workloads  # noqa: E402
from oracle.oracle import OrDct, OrTrainCfg, model_of, oracle, reference  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
SAVE_EVERY = 10   # iterations between saves of the loop's state

# workload -> (iterations, first FD iteration or None, checkpoint spacing, pairs or None = the workload's own)
SCHEDULES = {
    "rgb256": dict(iters=200, every=50),
    "rgb512_two_level": dict(iters=2000, every=250),
    "material512": dict(iters=1050, fd_from=1001, every=250, fp16_end=True),
    "dct512": dict(iters=4000, every=250, dct_start=2000, dct_refit=500, dct_refit_until=4000, dct_lambda=0.5, lo16=4,
                   shadow_pull=0.01),
    "material2048": dict(iters=10, every=5, pairs=64),
}


def inputs(w):
    lay = w.layout
    maps = synth.material(w.seed, lay.W, lay.H) if lay.T == 4 else [synth.rgb_texture(w.seed, lay.W, lay.H)]
    tgt = synth.target_from_maps(maps)
    z, p = synth.init_model(lay, w.seed, qat_bits=w.qat_bits)
    return z, p, tgt


def digest(*arrays) -> np.ndarray:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return np.frombuffer(h.digest(), np.uint8).copy()


def mse_psnr(orc, img, tgt, lay):
    """mse_of (main.cpp:1764-1788: both images rounded to 8 bits, per-texture weights) and 10 log10(255^2 / mse)"""
    tex, weighted = np.zeros(4), np.zeros(1)
    wv = np.array([float(x) for x in (lay.weights or [1.0] * lay.T)], np.float32)
    orc._mse_of(img.ctypes.data, tgt.ctypes.data, lay.W, lay.H, lay.nout, wv.ctypes.data, float(np.float32(wv.sum())), 0, 0,
                tex.ctypes.data, weighted.ctypes.data)
    mse = float(weighted[0])
    return mse, 10 * math.log10(255.0 ** 2 / mse)


def dct_state(w, lam, lo16):
    """the DCT level's host tables: steps at the workload's quality, lambda weights, empty codes and symbols"""
    W0, H0, C0, _ = w.layout.levels[0]
    n = (W0 // 8) * (H0 // 8) * C0
    t16, _ = dct_host.lambda_weights(lam, w.layout.W, w.layout.H, True, True)
    h = {"steps": np.concatenate([dct_host.steps(q, 4).reshape(-1) for q in w.dct_q]).astype(np.int32),
         "code": np.zeros(n, np.uint8), "sym": np.zeros(n * 64, np.int16)}
    d = OrDct()
    d.C, d.BW, d.BH, d.dc_step, d.deadzone, d.lo_w16 = C0, W0 // 8, H0 // 8, 4, 0, lo16
    for k in range(16):
        d.lam_t16[k] = t16[k]
    d.step = h["steps"].ctypes.data_as(C.POINTER(C.c_int))
    d.code = h["code"].ctypes.data_as(C.POINTER(C.c_uint8))
    d.sym = h["sym"].ctypes.data_as(C.POINTER(C.c_int16))
    return d, h


def run(name: str, state_dir: str, isa: str = "x86-64-v3"):
    w = workloads()[name]
    s = SCHEDULES[name]
    lay = w.layout
    iters, every = s["iters"], s["every"]
    fd_from = s.get("fd_from") or iters + 1
    pairs = s.get("pairs") or w.mlp_pairs
    z, p, tgt = inputs(w)
    orc = oracle()
    ref = reference(fast=True, isa=isa)
    L = ref.lib
    cfg = OrTrainCfg()
    cfg.seed, cfg.mlp_pairs, cfg.mlp_batch, cfg.mlp_sigma, cfg.mlp_lr = w.seed, pairs, w.mlp_batch, w.mlp_sigma, w.mlp_lr
    cfg.lat_pairs, cfg.lat_sigma, cfg.lat_lr, cfg.fd_from, cfg.fd_h = w.lat_pairs, w.lat_sigma, w.lat_lr, fd_from, w.fd_h
    cfg.qat = max(w.qat_bits) if w.qat_bits else 0
    for c, b in enumerate(w.qat_bits or []):
        cfg.qat_ch[c] = b
    mc = model_of(lay)
    keep = None
    if w.dct_q:
        d, keep = dct_state(w, s["dct_lambda"], s["lo16"])
        h = L.ref_train_create_dct_sched(C.byref(mc), C.byref(cfg), z.ctypes.data, p.ctypes.data, tgt.ctypes.data, C.byref(d),
                                         C.c_float(s["dct_lambda"]), 1, 1, s["dct_start"], s["dct_refit"], s["dct_refit_until"])
        L.ref_train_set_shadow_pull(h, C.c_float(s["shadow_pull"]))
    else:
        h = L.ref_train_create(C.byref(mc), C.byref(cfg), z.ctypes.data, p.ctypes.data, tgt.ctypes.data)
    os.makedirs(state_dir, exist_ok=True)
    tag = digest(z, p, tgt).tobytes().hex()[:16] + ("" if isa == "x86-64-v3" else "_" + isa)
    spath = os.path.join(state_dir, f"{name}_{tag}.state")
    jpath = os.path.join(state_dir, f"{name}_{tag}.json")
    log = {"checkpoints": [], "psnr": [], "mse": [], "done": 0, "seconds": 0.0}
    if os.path.exists(jpath) and os.path.exists(spath) and L.ref_train_load(h, spath.encode()):
        with open(jpath) as f:
            log = json.load(f)
        print(f"{name}: resumed after iteration {log['done']}", flush=True)
    zb, pb = np.empty_like(z), np.empty_like(p)

    def measure():
        L.ref_train_get_zdec(h, zb.ctypes.data)
        L.ref_train_get(h, None, pb.ctypes.data)
        return mse_psnr(orc, orc.decode_full(lay, pb, zb), tgt, lay)

    mse0, ps0 = mse_psnr(orc, orc.decode_full(lay, p, z), tgt, lay)
    t0 = time.time() - log["seconds"]
    try:
        for it in range(log["done"] + 1, iters + 1):
            L.ref_train_iter(h, it, iters)
            if it % every == 0 and it != iters:
                mse, ps = measure()
                log["checkpoints"].append(it); log["mse"].append(mse); log["psnr"].append(ps)
                print(f"{name}: iteration {it}: psnr {ps:.4f} dB ({time.time() - t0:.0f} s)", flush=True)
            if it % SAVE_EVERY == 0 and it != iters:
                log["done"], log["seconds"] = it, time.time() - t0
                if not L.ref_train_save(h, (spath + ".tmp").encode()):
                    raise RuntimeError(f"cannot write {spath}")
                with open(jpath + ".tmp", "w") as f:
                    json.dump(log, f)
                os.replace(spath + ".tmp", spath)
                os.replace(jpath + ".tmp", jpath)
        if s.get("fp16_end"):
            if not L.ref_train_round_fp16(h):
                raise RuntimeError("a weight has no fp16 value")
        mse_f, ps_f = measure()
        out = dict(workload=np.array(name), digest=digest(z, p, tgt), iters=np.int32(iters), fd_from=np.int32(fd_from),
                   pairs=np.int32(pairs), fp16_end=np.int32(bool(s.get("fp16_end"))), checkpoints=np.array(log["checkpoints"], np.int32),
                   psnr=np.array(log["psnr"]), mse=np.array(log["mse"]), start_psnr=np.float64(ps0), start_mse=np.float64(mse0),
                   final_psnr=np.float64(ps_f), final_mse=np.float64(mse_f), cpu_seconds=np.float64(time.time() - t0),
                   threads=np.int32(L.ref_omp_threads()), isa=np.array(isa))
        if w.dct_q:
            code = np.zeros(keep["code"].size, np.uint8)
            L.ref_train_get_dct_codes(h, code.ctypes.data)
            out.update(dct_start=np.int32(s["dct_start"]), dct_refit=np.int32(s["dct_refit"]),
                       dct_refit_until=np.int32(s["dct_refit_until"]), dct_lambda=np.float32(s["dct_lambda"]),
                       lo16=np.int32(s["lo16"]), shadow_pull=np.float32(s["shadow_pull"]), final_codes=code)
        path = os.path.join(OUT, f"final_psnr_{name}{'' if isa == 'x86-64-v3' else '_' + isa.split('-')[-1]}.npz")
        np.savez_compressed(path, **out)
        print(f"{name}: {iters} iterations, start psnr {ps0:.4f} dB, final psnr {ps_f:.4f} dB (mse {mse_f:.4f}), "
              f"{time.time() - t0:.0f} s -> {os.path.relpath(path, ROOT)}", flush=True)
    finally:
        L.ref_train_destroy(h)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("workloads", nargs="+", choices=sorted(SCHEDULES))
    ap.add_argument("--state", default=os.path.join(tempfile.gettempdir(), "ntc_final_psnr"),
                    help="where the loop's state is kept between checkpoints")
    ap.add_argument("--isa", default="x86-64-v3", choices=["x86-64-v3", "x86-64-v4"],
                    help="the reference build (its own -O3 -ffast-math flags) for this x86-64 level; the fixtures the "
                         "tests hold to their bars are the x86-64-v3 build's, an x86-64-v4 run (final_psnr_<workload>_v4.npz) "
                         "measures how far two builds of the reference's own loop end apart")
    a = ap.parse_args()
    for name in a.workloads:
        run(name, a.state, a.isa)


if __name__ == "__main__":
    main()
