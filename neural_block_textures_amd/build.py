"""Build recipe of libntc_hip.so (in-tree, for gfx950) with hipcc.

    python -m neural_block_textures_amd.build        # or __graft_entry__.build()

Every translation unit is compiled for gfx950 with FMA contraction off (the kernels write each
fused multiply-add explicitly) and without packed-FP32 instructions; objects are rebuilt in
parallel and linked into neural_block_textures_amd/libntc_hip.so.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libntc_hip.so")
SOURCES = ["kernels_pop.hip", "kernels_mlp.hip", "kernels_latent.hip", "kernels_quant.hip", "kernels_stats.hip", "noalloc.hip", "trainer.cpp",
           "noise_fix.cpp", "capi.cpp", "jit.cpp"]
ARCH = "gfx950"
# The matrix-core population evaluation takes maxima of values that are never NaN for a finite
# model (the reference's own build assumes no NaNs either, -ffast-math): with the IEEE mode bit
# off, v_max_f32 needs no canonicalising copies of its operands.
EXTRA = {"kernels_pop.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libntc_hip.so)")


def flags(src: str) -> list[str]:
    f = ["-std=c++17", "-O3", "-fPIC", f"-I{INCLUDE}", f"-I{CSRC}", "-ffp-contract=off", "-Wall", "-Wno-unused-function",
         "-Wno-unused-result", "-Wno-unknown-pragmas"]
    if src.endswith(".hip"):
        f += [f"--offload-arch={ARCH}", "-x", "hip", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
              "-munsafe-fp-atomics",
              # matrix-core results straight into VGPRs: no AGPR copies between a layer and its activation
              "-mllvm", "-amdgpu-mfma-vgpr-form"]
    else:
        f += ["-D__HIP_PLATFORM_AMD__"]
    return f + EXTRA.get(src, [])


def build(verbose: bool = False, jobs: int = 4) -> str:
    os.makedirs(BUILD, exist_ok=True)
    cc = hipcc()
    objs = []

    def compile_one(src):
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
        cmd = [cc, *flags(src), "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"compiling {src} failed:\n{r.stdout}\n{r.stderr}")
        if r.stderr.strip() and verbose:
            print(r.stderr, file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [cc, "-shared", f"--offload-arch={ARCH}", "-o", tmp, *objs, "-lpthread", "-lhiprtc", "-ldl"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"linking libntc_hip.so failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
