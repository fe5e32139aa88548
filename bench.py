#!/usr/bin/env python3
"""Benchmark: ES training iterations of the benchmark workloads on one MI355X, with the
reference's OpenMP CPU path timed beside them.

A step is one ES iteration of the reference's per-iteration call sequence (main.cpp:4121-4148):
MLP ES step, latent ES step, then the --qat selector search when the workload has one (a live
--dct-q level 0 re-snaps and adds its rate pass inside the latent step). Inputs are synthetic
(neural_block_textures_amd/synth.py) and resident on the device before timing starts.

    python bench.py [--steps K] [--warmup W] [--workload material512]
    python bench.py --all-configs profiles/es_iterations_all_configs.md

Untimed iterations run for --settle seconds (default 1) before the W warm-up steps, so that the K timed steps see
the steady state of a training run rather than a process's first iterations. The default run prints one JSON line
for material512. value = every member-pixel MLP evaluation
of the timed iterations (population, latent pairs, selector search) per second of wall time;
roofline = the population-evaluation kernel's algorithmic FP32 FLOP per launch over its mean launch
time (HIP events on the trainer's stream), against the MI355X FP32 peak. --all-configs runs each of
the five workloads (GPU ES iterations/s and a bounded sample of the reference's CPU loop) and
writes a table.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP32_PEAK_TFLOPS = 157.3
VALU_F32_PEAK_TFLOPS = 78.6   # one FP32 FMA per lane per cycle (no packed instructions)
METRIC = "member·pixel evals/sec + ES iterations/sec (512² 4-tex, pop 8192), % roofline"
KERNELS = ("batch", "perturb", "pop_eval", "es_grad", "adam", "lat_eps", "lat_pair", "lat_gather", "qat_search", "decode",
           "fd_sets", "qes_snap", "dct_snap", "dct_rate", "shadow_pull")
DCT_CODE = 8          # the scale code set before the first device refit replaces it with the probe's
DCT_LAMBDA = 0.5      # the reference's default --dct-lambda at q 50: min(0.5, 7.5 S(q)^2)
DCT_LO16 = 4          # the default --dct-lambda-lo 0.25 as round(16 W)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def macs(layout) -> int:
    w = [layout.nin] + list(layout.hidden) + [layout.nout]
    return sum(w[i] * w[i + 1] for i in range(len(w) - 1))


def evals_per_iter(w, pairs=None) -> dict:
    lay = w.layout
    npix = lay.W * lay.H
    active = [l for l in range(len(lay.levels)) if not (w.qat_bits and l == 0)]
    e = {"population": 2 * (pairs or w.mlp_pairs) * w.mlp_batch, "latent": 2 * w.lat_pairs * npix if active else 0,
         "qat": sum(1 << b for b in w.qat_bits) * npix if w.qat_bits else 0}
    e["total"] = sum(e.values())
    return e


def inputs(w):
    from neural_block_textures_amd import synth
    lay = w.layout
    maps = synth.material(w.seed, lay.W, lay.H) if lay.T == 4 else [synth.rgb_texture(w.seed, lay.W, lay.H)]
    tgt = synth.target_from_maps(maps)
    z, p = synth.init_model(lay, w.seed, qat_bits=w.qat_bits)
    return z, p, tgt


def dct_host_state(w, codes=None):
    """codes (default: the constant DCT_CODE), symbols, steps, lambda weights of the workload's DCT-coded level 0"""
    import numpy as np

    from neural_block_textures_amd import dct_host
    W0, H0, C0, _ = w.layout.levels[0]
    n = (W0 // 8) * (H0 // 8) * C0
    t16, scale = dct_host.lambda_weights(DCT_LAMBDA, w.layout.W, w.layout.H, True, True)
    code = np.full(n, DCT_CODE, np.uint8) if codes is None else np.ascontiguousarray(codes, np.uint8).copy()
    return {"C": C0, "BW": W0 // 8, "BH": H0 // 8, "n": n, "code": code,
            "sym": np.zeros(n * 64, np.int16), "steps": np.concatenate([dct_host.steps(q, 4).reshape(-1) for q in w.dct_q]),
            "lam_t16": t16, "rate_scale": scale}


MATRIX_CORES = [True]   # False: every stage on the VALU kernels (--valu)
POP_SAMPLE = 8          # the timed region times one population launch in this many


def make_trainer(w, z, p, tgt):
    from neural_block_textures_amd import dct_host, synth
    from neural_block_textures_amd.trainer import DctDesc, Trainer
    lay = w.layout
    kw = dict(max_pairs=w.mlp_pairs, max_batch=w.mlp_batch, seed=w.seed)
    if w.qat_bits:
        kw.update(qat_bits=w.qat_bits, qat_grid=synth.qat_grid())
    if w.dct_q:
        kw.update(dct={"C": lay.levels[0][2], "q": w.dct_q, "dc_step": 4}, dct_basis=dct_host.basis(),
                  dct_zigzag=dct_host.zigzag())
    tr = Trainer()
    tr.init(Trainer.model_desc(lay, **kw), z, p, tgt, lay)
    if not MATRIX_CORES[0]:
        tr.set_matrix_cores(False)
    if w.dct_q:
        h = dct_host_state(w)
        d = DctDesc()
        d.live, d.C, d.BW, d.BH, d.N, d.dc_step = 1, h["C"], h["BW"], h["BH"], 8, 4
        d.rate_es, d.rate_trunc, d.rate_scale = 1, 1, h["rate_scale"]
        for k in range(16):
            d.lam_t16[k] = h["lam_t16"][k]
        d.lo_w16, d.deadzone = DCT_LO16, 0
        tr.set_dct(d, h["code"], h["sym"], h["steps"])
        tr.dct_codes = tr.dct_refit()   # the scale codes from the decoder sensitivity probe, as at the reference's DCT switch
        tr.dct_desc = d
    return tr


def es_iter(tr, w, it):
    tr.mlp_step(it, w.mlp_sigma, w.mlp_lr, w.mlp_pairs, w.mlp_batch)
    tr.lat_step(it, w.lat_sigma, w.lat_lr, w.lat_pairs)
    if w.dct_q and w.shadow_pull > 0:   # the live plane's shadow pulled toward it and re-snapped (main.cpp:4136)
        W0, H0, C0, _ = w.layout.levels[0]
        tr.shadow_pull(0, W0 * H0 * C0, w.shadow_pull)
    if w.qat_bits:
        tr.qat_search()


def cpu_baseline(w, z, p, tgt, seconds: float, pairs=None, dct_codes=None):
    """The reference's CPU training loop (main.cpp compiled with its own -O3 -ffast-math flags and
    OpenMP, oracle/_ref/libntc_ref_fast.so) on the same inputs for a bounded number of iterations
    (with `pairs` < the workload's population for a sample of a very large one); the oracle's
    restatement where the reference build is absent."""
    import numpy as np

    from oracle import oracle as O
    mc = O.model_of(w.layout)
    cfg = O.OrTrainCfg()
    pairs = pairs or w.mlp_pairs
    cfg.seed, cfg.mlp_pairs, cfg.mlp_batch, cfg.mlp_sigma, cfg.mlp_lr = w.seed, pairs, w.mlp_batch, w.mlp_sigma, w.mlp_lr
    cfg.lat_pairs, cfg.lat_sigma, cfg.lat_lr = w.lat_pairs, w.lat_sigma, w.lat_lr
    cfg.qat = max(w.qat_bits) if w.qat_bits else 0
    for c, b in enumerate(w.qat_bits or []):
        cfg.qat_ch[c] = b
    cfg.fd_from, cfg.fd_h = w.iters + 1, w.fd_h
    ev = evals_per_iter(w, pairs)["total"]
    keep = []
    isa = None
    if O.have_reference(fast=True):
        isa = O.host_isa()
        ref_path = O.reference_path(fast=True, isa="auto")   # the widest build the host supports (-march=native's choice)
        L = O.reference(fast=True, isa="auto").lib
        if w.dct_q:
            h = dct_host_state(w, dct_codes)
            d = O.OrDct()
            d.C, d.BW, d.BH, d.dc_step, d.deadzone, d.lo_w16 = h["C"], h["BW"], h["BH"], 4, 0, DCT_LO16
            for k in range(16):
                d.lam_t16[k] = h["lam_t16"][k]
            keep = [h["steps"], h["code"], h["sym"]]
            d.step = h["steps"].ctypes.data_as(C.POINTER(C.c_int))
            d.code = h["code"].ctypes.data_as(C.POINTER(C.c_uint8))
            d.sym = h["sym"].ctypes.data_as(C.POINTER(C.c_int16))
            hnd = L.ref_train_create_dct(C.byref(mc), C.byref(cfg), z.ctypes.data, p.ctypes.data, tgt.ctypes.data, C.byref(d),
                                         DCT_LAMBDA, 1, 1)
        else:
            hnd = L.ref_train_create(C.byref(mc), C.byref(cfg), z.ctypes.data, p.ctypes.data, tgt.ctypes.data)
        threads = L.ref_omp_threads()
        step = lambda it: L.ref_train_iter(hnd, it, w.iters)
        kind = "reference"
    else:
        if w.dct_q:
            return None
        orc = O.oracle()
        st = O.OrTrainState()
        arrs = [z.copy(), p.copy()] + [np.zeros_like(a) for a in (p, p, z, z)]
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
        L.ref_train_destroy(hnd)
    del keep
    sample = f"{its} ES iteration(s) of {w.name} (the full per-iteration sequence at full size), {el:.1f} s"
    if pairs != w.mlp_pairs:
        sample = (f"{its} ES iteration(s) of {w.name} with {pairs} of its {w.mlp_pairs} pairs (population evaluation scaled "
                  f"down, everything else at full size), {el:.1f} s")
    out = {"value": ev * its / el, "unit": "member·pixel evals/s", "cores": threads, "kind": kind, "sample": sample,
           "es_iters_per_s": its / el, "cpu": cpu_model(), "cpuid": cpu_ids(), "nproc": os.cpu_count(),
           "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None}
    if kind == "reference":
        out["isa"] = isa
        out["build"] = f"{os.path.relpath(ref_path, ROOT)} (-O3 -ffast-math -fopenmp -march=" + \
            ("x86-64-v4" if ref_path.endswith("_v4.so") else "x86-64-v3") + ")"
    return out


def gauss_draw(w, reps: int):
    """The device draw of all N x P Gaussians of one ES step of the workload (Trainer.debug_gauss, the population
    kernel's per-element draw), reps times, timed with HIP events on the trainer's stream."""
    import numpy as np

    from neural_block_textures_amd import synth
    from neural_block_textures_amd.trainer import Trainer
    lay = w.layout
    z, p = synth.init_model(lay, w.seed, qat_bits=w.qat_bits)
    tr = Trainer()
    kw = dict(qat_bits=w.qat_bits, qat_grid=synth.qat_grid()) if w.qat_bits else {}
    tr.init(Trainer.model_desc(lay, max_pairs=8, max_batch=256, seed=w.seed, **kw), z, p,
            np.zeros(lay.W * lay.H * lay.nout, np.float32), lay)
    n = w.mlp_pairs * lay.nparams
    t0 = time.perf_counter()
    for _ in range(reps):
        g = tr.debug_gauss(2, 1, 0, 0, n)   # includes the download of the n values
    el = time.perf_counter() - t0
    print(json.dumps({"gauss_draw": {"workload": w.name, "gaussians": n, "reps": reps, "host_ms_per_draw_with_download": 1e3 * el / reps,
                                     "mean": float(g.mean()), "std": float(g.std())}}), flush=True)
    tr.close()


def cpu_model() -> str:
    """the host CPU's model name (/proc/cpuinfo), else the architecture"""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_ids() -> dict:
    """/proc/cpuinfo's vendor, family, model and stepping numbers of the first CPU, and its AVX-512 flags"""
    out = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k in ("vendor_id", "cpu family", "model", "stepping", "microcode"):
                    out[k.replace(" ", "_")] = v
                elif k == "flags":
                    out["avx512"] = sorted(x for x in v.split() if x.startswith("avx512"))
    except OSError:
        pass
    return out


def cpu_refit_ms(w, r):
    """The reference's host refit of the same state (main.cpp:4110-4120 with --cuda: the model downloaded,
    dct_probe_codes and the level-0 snap on the host's cores; the set_dct upload not included)."""
    import numpy as np

    from oracle import oracle as O
    if not O.have_reference(fast=True):
        return None
    L = O.reference(fast=True, isa="auto").lib
    (z, p), zq = r["host_state"]
    h = dct_host_state(w, r["dct_codes"])
    d = O.OrDct()
    d.C, d.BW, d.BH, d.dc_step, d.deadzone, d.lo_w16 = h["C"], h["BW"], h["BH"], 4, 0, DCT_LO16
    for k in range(16):
        d.lam_t16[k] = h["lam_t16"][k]
    d.step = h["steps"].ctypes.data_as(C.POINTER(C.c_int))
    d.code = h["code"].ctypes.data_as(C.POINTER(C.c_uint8))
    d.sym = h["sym"].ctypes.data_as(C.POINTER(C.c_int16))
    mc = O.model_of(w.layout)
    W0, H0, C0, _ = w.layout.levels[0]
    lv0 = O.OrLevel(W0, H0, C0, 1, 0)
    n0 = W0 * H0 * C0
    zs, zqo = z[:n0].copy(), np.zeros(n0, np.float32)
    t0 = time.perf_counter()
    L.ref_dct_probe_codes(C.byref(mc), p.ctypes.data, zq.ctypes.data, C.byref(d), h["code"].ctypes.data)
    L.ref_dct_snap_level0(C.byref(d), C.byref(lv0), zs.ctypes.data, zqo.ctypes.data, None, None)
    return 1e3 * (time.perf_counter() - t0)


def run_gpu(w, steps, warmup, fd_steps=0, seconds=0.0, settle=0.0):
    """GPU ES iterations of workload w; with seconds > 0 the step count is chosen to time about that long.

    settle: untimed iterations, in groups of 8, until this many seconds of wall time have passed, before the warm-up
    steps. On the MI355X the first hundred-odd material512 iterations of a process run slower than the later ones
    (population launch 1.022-1.034 ms after 5 warm-up iterations, 1.007 ms after 200), so a short timed region right
    after a short warm-up would time that start rather than the training loop's steady state."""
    import numpy as np
    z, p, tgt = inputs(w)
    tr = make_trainer(w, z, p, tgt)
    log(f"bench: {w.name}:", tr.banner())
    it = 0
    settle_iters = 0
    t_settle = time.perf_counter()
    while time.perf_counter() - t_settle < settle:
        for _ in range(8):
            it += 1
            es_iter(tr, w, it)
        settle_iters += 8
        tr.synchronize()
    for _ in range(warmup):
        it += 1
        es_iter(tr, w, it)
    tr.synchronize()
    if seconds > 0:
        t0 = time.perf_counter()
        for _ in range(2):
            it += 1
            es_iter(tr, w, it)
        tr.synchronize()
        per = (time.perf_counter() - t0) / 2
        steps = int(min(2000, max(3, math.ceil(seconds / per))))
    # the timed region: one launch of the population kernel in POP_SAMPLE timed by HIP events on the trainer's
    # stream, recorded by the launch itself (a timed launch still costs the stream about 11 us on the
    # MI355X - 6.7 before it and 4.5 after, in a kernel trace of material512 - so timing every launch would
    # slow the region it measures; the other launches go untimed)
    tr.set_profiling(True, only=["pop_eval"], every=POP_SAMPLE)
    tr.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        it += 1
        es_iter(tr, w, it)
    tr.synchronize()
    el = time.perf_counter() - t0
    pop_ms, pop_n = tr.kernel_time("pop_eval")
    tr.set_profiling(False)
    # the per-kernel breakdown: a further profiled stretch with every launch bracketed
    tr.set_profiling(True)
    for _ in range(max(3, min(steps, 50))):
        it += 1
        es_iter(tr, w, it)
    tr.synchronize()
    kernels = {}
    for name in KERNELS:
        ms, n = tr.kernel_time(name)
        if n:
            kernels[name] = {"ms_total": round(ms, 3), "launches": n, "ms_mean": round(ms / n, 4)}
    tr.set_profiling(False)
    if pop_n:   # the roofline's launch time is the timed region's
        kernels["pop_eval"] = {"ms_total": round(pop_ms, 3), "launches": pop_n, "ms_mean": round(pop_ms / pop_n, 4)}
    fd = None
    if fd_steps > 0:
        def fd_iter():
            tr.mlp_step_fd(it, np.float32(w.fd_h), w.mlp_lr, w.mlp_batch)
            tr.lat_step(it, w.lat_sigma, w.lat_lr, w.lat_pairs)
            if w.qat_bits:
                tr.qat_search()
        tr.reset_mlp_adam()
        it += 1
        fd_iter()   # the first step sizes the weight-set buffer
        tr.set_profiling(True, only=["pop_eval"], every=POP_SAMPLE)
        tr.synchronize()
        t1 = time.perf_counter()
        for _ in range(fd_steps):
            it += 1
            fd_iter()
        tr.synchronize()
        fd_el = time.perf_counter() - t1
        fd_pop_ms, fd_pop_n = tr.kernel_time("pop_eval")
        tr.set_profiling(False)
        fd = {"iters_per_s": fd_steps / fd_el, "ms_per_iter": 1e3 * fd_el / fd_steps,
              "evals_per_s": (2 * (w.layout.nparams + 1) * w.mlp_batch) * fd_steps / fd_el,
              "pop_eval_ms": round(fd_pop_ms / max(fd_pop_n, 1), 4),
              "pop_kernel": "k_pop_mfma" if tr.on_matrix_cores("pop_eval") else "k_pop_eval"}
    refit = None
    if w.dct_q:   # the device refit (probe + re-snap) against the reference's host path for the same step
        tr.synchronize()
        t1 = time.perf_counter()
        for _ in range(5):
            tr.dct_refit()
        wall = 1e3 * (time.perf_counter() - t1) / 5
        tr.set_profiling(True)
        for _ in range(5):
            tr.dct_refit()
        tr.synchronize()
        kms = sum(tr.kernel_time(k)[0] for k in ("dct_probe", "dct_snap", "qes_snap"))
        tr.set_profiling(False)
        refit = {"device_ms": kms / 5, "with_download_ms": wall}
    loss, _ = tr.mlp_stats()
    img = tr.decode_full()
    assert np.isfinite(img).all() and np.isfinite(loss)
    name = "k_pop_eval"
    if tr.on_matrix_cores("pop_eval"):
        name = ("k_pop_pair_own" if tr.on_matrix_cores("pop_pair_own") else "k_pop_pair") if tr.on_matrix_cores("pop_pair") else "k_pop_mfma"
    out = {"z": z, "p": p, "tgt": tgt, "steps": steps, "el": el, "kernels": kernels, "fd": fd, "loss": loss, "pop_kernel": name,
           "refit": refit, "dct_codes": getattr(tr, "dct_codes", None), "settle": {"seconds": settle, "iterations": settle_iters}}
    if w.dct_q:
        out["host_state"] = (tr.download_model(), tr.download_zq())
    tr.close()
    return out


def roofline_of(w, r):
    ev = evals_per_iter(w)
    pe = r["kernels"]["pop_eval"]
    pop_flop = ev["population"] * 2 * macs(w.layout)
    achieved = pop_flop / (pe["ms_mean"] * 1e-3) / 1e12
    # the VALU kernels (--valu) against the FP32 VALU peak without packed instructions
    bound, peak = ("mfma", FP32_PEAK_TFLOPS) if r["pop_kernel"] != "k_pop_eval" else ("valu", VALU_F32_PEAK_TFLOPS)
    roof = {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4), "traffic": None, "kernel": r["pop_kernel"],
            "flop_per_launch": pop_flop, "ms_per_launch": pe["ms_mean"]}
    # HBM bytes per launch from the committed counter runs (FETCH_SIZE and WRITE_SIZE, each scaled by the
    # same counter's reading for a plain copy of known size): profiles/traffic_<workload>.json
    tpath = os.path.join(ROOT, "profiles", f"traffic_{w.name}.json")
    if os.path.exists(tpath) and bound == "mfma":
        with open(tpath) as f:
            t = json.load(f)
        if t.get("pop_eval_kernel", "").startswith(r["pop_kernel"] + "<"):   # counters of the kernel that ran
            roof["traffic"] = t.get("pop_eval_bytes_per_launch")
            roof["traffic_source"] = os.path.relpath(tpath, ROOT)
    return roof


def all_configs(out_path: str, cpu_seconds: float):
    from neural_block_textures_amd.configs import workloads
    rows = []
    for name, w in workloads().items():
        r = run_gpu(w, 0, 3, seconds=2.0, settle=1.0)
        gpu_its = r["steps"] / r["el"]
        ev = evals_per_iter(w)
        # a population too large for a bounded CPU sample (over about 4 TFLOP per iteration) is sampled with 64 pairs
        pairs = w.mlp_pairs if ev["total"] * 2 * macs(w.layout) < 4e12 else 64
        log(f"bench: {name}: GPU {gpu_its:.2f} it/s; CPU sample ...")
        cpu = cpu_baseline(w, r["z"], r["p"], r["tgt"], cpu_seconds, pairs=pairs, dct_codes=r["dct_codes"]) if cpu_seconds > 0 else None
        if r["refit"] is not None and cpu_seconds > 0:
            r["refit"]["host_ms"] = cpu_refit_ms(w, r)
        cpu_its = cpu["value"] / ev["total"] if cpu else None   # full-size iterations per second at the sampled rate
        row = {"workload": name, "gpu_es_iters_per_s": gpu_its, "gpu_ms_per_iter": 1e3 / gpu_its, "gpu_steps": r["steps"],
               "gpu_evals_per_s": ev["total"] * gpu_its, "evals_per_iter": ev, "roofline": roofline_of(w, r),
               "kernels": r["kernels"], "cpu": cpu, "cpu_es_iters_per_s": cpu_its,
               "speedup": gpu_its / cpu_its if cpu_its else None, "dct_refit": r["refit"]}
        print(json.dumps(row), flush=True)
        rows.append(row)
    with open(out_path, "w") as f:
        f.write("# ES iterations per second, all five workloads (one MI355X vs the reference's CPU loop)\n\n")
        f.write("Command (from the repository root on the MI355X box):\n\n```\n" + " ".join(["python3"] + sys.argv) + "\n```\n\n")
        f.write("| workload | GPU ES it/s | GPU ms/iter | member-pixel evals/iter | population kernel | TFLOP/s | % of 157.3 "
                "| CPU ES it/s | CPU threads, ISA | speedup | CPU sample |\n|---|---|---|---|---|---|---|---|---|---|---|\n")
        for row in rows:
            c = row["cpu"] or {}
            rf = row["roofline"]
            f.write(f"| {row['workload']} | {row['gpu_es_iters_per_s']:.2f} | {row['gpu_ms_per_iter']:.3f} | "
                    f"{row['evals_per_iter']['total']:,} | `{rf['kernel']}` {rf['ms_per_launch']:.4f} ms | {rf['achieved']:.1f} | "
                    f"{100 * rf['frac']:.1f}% | {row['cpu_es_iters_per_s'] or 0:.3g} | {c.get('cores', '-')}, {c.get('isa') or c.get('kind', '-')} | "
                    f"{row['speedup'] or 0:.0f}x | {c.get('sample', '-')} |\n")
        f.write("\nKernel launches per ES iteration (HIP events around every launch of a further profiled stretch of the same run; "
                "mean ms per launch x launches per iteration):\n\n| workload | " + " | ".join(KERNELS) + " |\n|---|" + "---|" * len(KERNELS) + "\n")
        for row in rows:
            ks = row["kernels"]
            iters = max(1, ks.get("es_grad", ks.get("batch", {"launches": 1}))["launches"])
            cells = []
            for name in KERNELS:
                k = ks.get(name)
                cells.append(f"{k['ms_mean']:.4f} x {k['launches'] / iters:g}" if k and name != "pop_eval" else
                             (f"{k['ms_mean']:.4f} x 1" if k else "-"))
            f.write(f"| {row['workload']} | " + " | ".join(cells) + " |\n")
        c = next((row["cpu"] for row in rows if row["cpu"]), None)
        if c:
            ids = c.get("cpuid") or {}
            f.write(f"\nCPU baseline host: {c.get('cpu')} (cpuinfo family {ids.get('cpu_family', '?')}, model {ids.get('model', '?')}), "
                    f"{c.get('nproc')} logical CPUs, {c.get('affinity_cpus')} in the affinity set; the reference's loop "
                    f"{c.get('build', '(the oracle restatement)')}, the widest build the host supports.\n")
        for row in rows:
            rf = row.get("dct_refit")
            if rf:
                f.write(f"\n{row['workload']}: a --dct-q refit (decoder sensitivity probe + level-0 re-snap) takes "
                        f"{rf['device_ms']:.3f} ms of kernels on the device ({rf.get('with_download_ms', 0):.3f} ms per call with the codes' "
                        f"download, `ntc_trainer_dct_refit`); the reference's host probe and snap "
                        f"of the same state take {rf.get('host_ms') or 0:.1f} ms on the host's cores (plus the model download "
                        f"and the set_dct upload).\n")
    log(f"bench: wrote {out_path}")


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="material512")
    ap.add_argument("--fd-steps", type=int, default=5, help="extra timed --mlp-fd iterations, reported apart")
    ap.add_argument("--settle", type=float, default=1.0, metavar="SECONDS",
                    help="untimed iterations for this long before the warm-up steps (steady-state clocks; 0 = none)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="bounded CPU-baseline sample (0 = skip)")
    ap.add_argument("--all-configs", metavar="OUT_MD", help="run the five workloads and write a table")
    ap.add_argument("--valu", action="store_true",
                    help="every stage on the VALU kernels (the same work; measures the matrix-core choice against the alternative)")
    ap.add_argument("--gauss-draw", type=int, default=0, metavar="REPS",
                    help="time REPS device draws of one ES step's N x P Gaussians of the workload (what a regenerating update redraws)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="FLOATS",
                    help="only run a plain device copy of FLOATS floats three times (the reference for memory counters)")
    ap.add_argument("--mlp-batch", type=int, default=0, metavar="M",
                    help="analysis only: the workload with an M-slot minibatch instead of its own (the line's config records it)")
    args = ap.parse_args()
    MATRIX_CORES[0] = not args.valu
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU only (asked for {max(args.gpus, world)}): this backend has no multi-GPU path; "
              "the population would shard over pairs with one all-gather of the pair differences", file=sys.stderr)
        sys.exit(2)

    import numpy as np

    from neural_block_textures_amd import synth
    from neural_block_textures_amd.configs import workloads
    from neural_block_textures_amd.trainer import Layout, Trainer

    if args.copy_calibration:
        small = Layout(8, 8, [(8, 8, 4, False)], [16, 16])
        zc, pc = synth.init_model(small, 1)
        tc = Trainer()
        tc.init(Trainer.model_desc(small), zc, pc, np.zeros(8 * 8 * 3, np.float32), small)
        n = args.copy_calibration & ~3
        tc.debug_copy_calibration(n, 3)
        tc.close()
        print(json.dumps({"copy_calibration": {"floats": n, "bytes_read": 4 * n, "bytes_written": 4 * n, "reps": 3}}))
        return
    if args.all_configs:
        all_configs(args.all_configs, args.cpu_seconds)
        return
    if args.gauss_draw:
        gauss_draw(workloads()[args.workload], args.gauss_draw)
        return

    w = workloads()[args.workload]
    if args.mlp_batch:
        w.mlp_batch = args.mlp_batch
    lay = w.layout
    log(f"bench: {w.name} {lay.W}x{lay.H}x{lay.T} levels {lay.levels} mlp {lay.nin}->{lay.hidden}->{lay.nout} "
        f"pairs {w.mlp_pairs} batch {w.mlp_batch}")
    r = run_gpu(w, args.steps, args.warmup, fd_steps=args.fd_steps, settle=args.settle)
    cpu = None
    if args.cpu_seconds > 0:
        log(f"bench: CPU baseline for {args.cpu_seconds:.0f} s ...")
        cpu = cpu_baseline(w, r["z"], r["p"], r["tgt"], args.cpu_seconds)
    ev = evals_per_iter(w)
    el = r["el"]
    pe = r["kernels"]["pop_eval"]
    out = {
        "metric": METRIC,
        "value": ev["total"] * args.steps / el, "unit": "member·pixel evals/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": 1e3 * el / args.steps, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": w.name, "image": [lay.W, lay.H, lay.T], "levels": [list(l) for l in lay.levels],
                   "mlp": [lay.nin] + list(lay.hidden) + [lay.nout], "population": w.population,
                   "minibatch": w.mlp_batch, "lat_pairs": w.lat_pairs, "qat": w.qat_bits, "dct_q": w.dct_q},
        "es_iters_per_s": args.steps / el,
        "evals_per_iter": ev,
        "population_evals_per_s": ev["population"] / (pe["ms_mean"] * 1e-3),
        "roofline": roofline_of(w, r),
        "cpu_baseline": cpu,
        "fd_phase": r["fd"],
        "kernels": r["kernels"],
        "batch_loss": r["loss"],
        "settle": r["settle"],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
