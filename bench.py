#!/usr/bin/env python3
"""Benchmark: ES training iterations of one benchmark workload on one MI355X, with the
reference's OpenMP CPU path timed beside it.

A step is one ES iteration of the reference's per-iteration call sequence (main.cpp:4121-4148):
MLP ES step, latent ES step, then the --qat selector search when the workload has one. Inputs are
synthetic (neural_block_textures_amd/synth.py) and resident on the device before timing starts.

    python bench.py [--steps K] [--warmup W] [--workload material512]

Prints one JSON line. value = every member-pixel MLP evaluation of the timed iterations (population,
latent pairs, selector search) per second of wall time; roofline = the population-evaluation
kernel's algorithmic FP32 FLOP per launch over its mean launch time (HIP events on the trainer's
stream), against the MI355X FP32 peak.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP32_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def macs(layout) -> int:
    w = [layout.nin] + list(layout.hidden) + [layout.nout]
    return sum(w[i] * w[i + 1] for i in range(len(w) - 1))


def evals_per_iter(w) -> dict:
    lay = w.layout
    npix = lay.W * lay.H
    active = [l for l in range(len(lay.levels)) if not (w.qat_bits and l == 0)]
    e = {"population": 2 * w.mlp_pairs * w.mlp_batch, "latent": 2 * w.lat_pairs * npix if active else 0,
         "qat": sum(1 << b for b in w.qat_bits) * npix if w.qat_bits else 0}
    e["total"] = sum(e.values())
    return e


def cpu_model(lay):
    from oracle.oracle import model_of
    return model_of(lay)


def cpu_baseline(w, z, p, tgt, seconds: float):
    """The reference's CPU training loop (main.cpp compiled with its own -O3 -ffast-math flags and
    OpenMP, oracle/_ref/libntc_ref_fast.so) on the same inputs, for a bounded number of
    iterations; falls back to the oracle's restatement when the reference build is absent."""
    from oracle import oracle as O
    mc = cpu_model(w.layout)
    cfg = O.OrTrainCfg()
    cfg.seed, cfg.mlp_pairs, cfg.mlp_batch, cfg.mlp_sigma, cfg.mlp_lr = w.seed, w.mlp_pairs, w.mlp_batch, w.mlp_sigma, w.mlp_lr
    cfg.lat_pairs, cfg.lat_sigma, cfg.lat_lr = w.lat_pairs, w.lat_sigma, w.lat_lr
    cfg.qat = max(w.qat_bits) if w.qat_bits else 0
    for c, b in enumerate(w.qat_bits or []):
        cfg.qat_ch[c] = b
    cfg.fd_from, cfg.fd_h = w.iters + 1, w.fd_h
    ev = evals_per_iter(w)["total"]
    if O.have_reference(fast=True):
        ref = O.reference(fast=True)
        L = ref.lib
        h = L.ref_train_create(C.byref(mc), C.byref(cfg), z.ctypes.data, p.ctypes.data, tgt.ctypes.data)
        threads = L.ref_omp_threads()
        step = lambda it: L.ref_train_iter(h, it, w.iters)
        kind = "reference"
    else:
        orc = O.oracle()
        st = O.OrTrainState()
        arrs = [z.copy(), p.copy()] + [__import__("numpy").zeros_like(a) for a in (p, p, z, z)]
        F = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
        st.z, st.p, st.wm, st.wv, st.zm, st.zv = (F(a) for a in arrs)
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        step = lambda it: orc.lib.or_train_iter(C.byref(mc), C.byref(cfg), C.byref(st), tgt.ctypes.data, it, w.iters)
        kind = "port"
    t0 = time.perf_counter()
    its = 0
    while True:
        its += 1
        step(its)
        el = time.perf_counter() - t0
        if el >= seconds or its >= 1000:
            break
    if kind == "reference":
        L.ref_train_destroy(h)
    return {"value": ev * its / el, "unit": "member·pixel evals/s", "cores": threads, "kind": kind,
            "sample": f"{its} ES iteration(s) of {w.name} (the full per-iteration sequence at full size), {el:.1f} s",
            "es_iters_per_s": its / el, "cpu": platform.processor() or platform.machine()}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="material512")
    ap.add_argument("--fd-steps", type=int, default=5, help="extra timed --mlp-fd iterations, reported apart")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="bounded CPU-baseline sample (0 = skip)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="FLOATS",
                    help="only run a plain device copy of FLOATS floats three times (the reference for memory counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU only (asked for {max(args.gpus, world)}): this backend has no multi-GPU path; "
              "the population would shard over pairs with one all-gather of the pair differences", file=sys.stderr)
        sys.exit(2)

    import numpy as np

    from neural_block_textures_amd import synth
    from neural_block_textures_amd.configs import workloads
    from neural_block_textures_amd.trainer import Trainer

    w = workloads()[args.workload]
    lay = w.layout
    if args.copy_calibration:
        from neural_block_textures_amd.trainer import Layout
        small = Layout(8, 8, [(8, 8, 4, False)], [16, 16])
        zc, pc = synth.init_model(small, 1)
        tc = Trainer()
        tc.init(Trainer.model_desc(small), zc, pc, np.zeros(8 * 8 * 3, np.float32), small)
        n = args.copy_calibration & ~3
        tc.debug_copy_calibration(n, 3)
        tc.close()
        print(json.dumps({"copy_calibration": {"floats": n, "bytes_read": 4 * n, "bytes_written": 4 * n, "reps": 3}}))
        return
    log(f"bench: {w.name} {lay.W}x{lay.H}x{lay.T} levels {lay.levels} mlp {lay.nin}->{lay.hidden}->{lay.nout} "
        f"pairs {w.mlp_pairs} batch {w.mlp_batch}")
    maps = synth.material(w.seed, lay.W, lay.H) if lay.T == 4 else [synth.rgb_texture(w.seed, lay.W, lay.H)]
    tgt = synth.target_from_maps(maps)
    z, p = synth.init_model(lay, w.seed, qat_bits=w.qat_bits)
    tr = Trainer()
    tr.init(Trainer.model_desc(lay, max_pairs=w.mlp_pairs, max_batch=w.mlp_batch, seed=w.seed, qat_bits=w.qat_bits,
                               qat_grid=synth.qat_grid() if w.qat_bits else None), z, p, tgt, lay)
    log("bench:", tr.banner())

    def es_iter(it):
        tr.mlp_step(it, w.mlp_sigma, w.mlp_lr, w.mlp_pairs, w.mlp_batch)
        tr.lat_step(it, w.lat_sigma, w.lat_lr, w.lat_pairs)
        if w.qat_bits:
            tr.qat_search()

    it = 0
    for _ in range(args.warmup):
        it += 1
        es_iter(it)
    tr.synchronize()
    tr.set_profiling(True)
    tr.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        it += 1
        es_iter(it)
    tr.synchronize()
    el = time.perf_counter() - t0
    kernels = {}
    for name in ("batch", "perturb", "pop_eval", "es_grad", "adam", "lat_eps", "lat_pair", "lat_gather", "qat_search",
                 "decode", "fd_sets", "qes_snap", "dct_snap", "dct_rate"):
        ms, n = tr.kernel_time(name)
        if n:
            kernels[name] = {"ms_total": round(ms, 3), "launches": n, "ms_mean": round(ms / n, 4)}
    tr.set_profiling(False)
    fd = None
    if args.fd_steps > 0:
        tr.reset_mlp_adam()
        tr.synchronize()
        t1 = time.perf_counter()
        for _ in range(args.fd_steps):
            it += 1
            tr.mlp_step_fd(it, np.float32(w.fd_h), w.mlp_lr, w.mlp_batch)
            tr.lat_step(it, w.lat_sigma, w.lat_lr, w.lat_pairs)
            if w.qat_bits:
                tr.qat_search()
        tr.synchronize()
        fd_el = time.perf_counter() - t1
        fd = {"iters_per_s": args.fd_steps / fd_el, "ms_per_iter": 1e3 * fd_el / args.fd_steps,
              "evals_per_s": (2 * (lay.nparams + 1) * w.mlp_batch) * args.fd_steps / fd_el}
    loss, dstd = tr.mlp_stats()
    img = tr.decode_full()
    assert np.isfinite(img).all() and np.isfinite(loss)
    tr.close()

    ev = evals_per_iter(w)
    flop_per_eval = 2 * macs(lay)
    pe = kernels["pop_eval"]
    pop_flop = ev["population"] * flop_per_eval
    achieved = pop_flop / (pe["ms_mean"] * 1e-3) / 1e12
    roofline = {"bound": "mfma", "achieved": round(achieved, 3), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / FP32_PEAK_TFLOPS, 4), "traffic": None,
                "kernel": "k_pop_eval", "flop_per_launch": pop_flop, "ms_per_launch": pe["ms_mean"]}
    # HBM bytes per launch from the committed counter runs (FETCH_SIZE and WRITE_SIZE, each scaled by the
    # same counter's reading for a plain copy of known size): profiles/traffic_<workload>.json
    tpath = os.path.join(ROOT, "profiles", f"traffic_{w.name}.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            t = json.load(f)
        roofline["traffic"] = t.get("pop_eval_bytes_per_launch")
        roofline["traffic_source"] = os.path.relpath(tpath, ROOT)
    cpu = None
    if args.cpu_seconds > 0:
        log(f"bench: CPU baseline for {args.cpu_seconds:.0f} s ...")
        cpu = cpu_baseline(w, z, p, tgt, args.cpu_seconds)
    value = ev["total"] * args.steps / el
    out = {
        "metric": "member·pixel evals/sec + ES iterations/sec (512² 4-tex, pop 8192), % roofline",
        "value": value, "unit": "member·pixel evals/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": 1e3 * el / args.steps, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": w.name, "image": [lay.W, lay.H, lay.T], "levels": [list(l) for l in lay.levels],
                   "mlp": [lay.nin] + list(lay.hidden) + [lay.nout], "population": w.population,
                   "minibatch": w.mlp_batch, "lat_pairs": w.lat_pairs, "qat": w.qat_bits},
        "es_iters_per_s": args.steps / el,
        "evals_per_iter": ev,
        "population_evals_per_s": ev["population"] / (pe["ms_mean"] * 1e-3),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "fd_phase": fd,
        "kernels": kernels,
        "batch_loss": loss,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
