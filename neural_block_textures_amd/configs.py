"""The five benchmark workloads, restated in the reference's flags (main.cpp option names).

"Level 1" / "latent2" of the workload descriptions are the reference's level 0 (--latent) and
level 1 (--latent2). An antithetic population of P members is --mlp-pairs P/2. "ReLU" is
--leak 0 (the two workloads that do not name an activation keep the default leak 0.01), phi(u,v) is --pos uv, "hidden 32" is 32,32. Unstated settings take the reference's
defaults (main.cpp:137-151): --lat-pairs 4, --lat-sigma 0.05, --lat-lr 0.02, --mlp-lr 0.005,
--mlp-sigma 0.02, --mlp-batch 4096. Every run draws its noise from the counter RNG (--rng hash).
"""
from __future__ import annotations

from dataclasses import dataclass, field

from .trainer import Layout, PK_UV


@dataclass
class Workload:
    name: str
    layout: Layout
    mlp_pairs: int
    mlp_batch: int = 4096
    mlp_sigma: float = 0.02
    mlp_lr: float = 0.005
    lat_pairs: int = 4
    lat_sigma: float = 0.05
    lat_lr: float = 0.02
    iters: int = 1000
    qat_bits: list = None
    fd_iters: int = 0          # trailing --mlp-fd iterations
    fd_h: float = 1e-3
    dct_q: list = None         # --dct-q per level-0 channel
    shadow_pull: float = 0.0   # --dct-shadow-pull: after every latent step on a live DCT plane (main.cpp:4136, 4142-4146)
    fp16_end: bool = False     # --write-ntcb: weights rounded to fp16 at the end
    seed: int = 1
    textures: int = 1
    notes: str = ""

    @property
    def population(self) -> int:
        return 2 * self.mlp_pairs


def _rgb(W, H, levels, hidden, **kw):
    return Layout(W, H, levels, hidden, T=1, pos=[PK_UV], leak=0.0, **kw)


def workloads() -> dict:
    return {
        # CPU-reference plumbing run, 256x256 RGB, 64x64x4 bilinear, 16,16, population 64
        "rgb256": Workload("rgb256", _rgb(256, 256, [(64, 64, 4, False)], [16, 16]), mlp_pairs=32, mlp_batch=65536,
                           mlp_sigma=0.01, iters=200, seed=11,
                           notes="full-image loss read as a 65536-slot minibatch drawn with replacement"),
        # 512x512 RGB, 128x128x8 + 32x32x4 bilinear, 32,32, population 1024 over 64K-pixel batches
        "rgb512_two_level": Workload("rgb512_two_level",
                                     _rgb(512, 512, [(128, 128, 8, False), (32, 32, 4, False)], [32, 32]),
                                     mlp_pairs=512, mlp_batch=65536, iters=2000, seed=12,
                                     notes="post-hoc 8-bit latent quantization is a host statistic"),
        # 4 x 512x512 material, --qat 2 512x512x2 nearest + 128x128x4 bilinear, 32,32, population 8192
        "material512": Workload("material512",
                                Layout(512, 512, [(512, 512, 2, True), (128, 128, 4, False)], [32, 32], T=4,
                                       pos=[PK_UV], leak=0.01),
                                mlp_pairs=4096, mlp_batch=4096, iters=8000, qat_bits=[2, 2], fd_iters=50,
                                fp16_end=True, seed=13, textures=4),
        # 512x512 RGB, --dct-q 50 plane 512x512x1 + 128x128x4, 32,32, population 4096
        "dct512": Workload("dct512", Layout(512, 512, [(512, 512, 1, True), (128, 128, 4, False)], [32, 32], T=1,
                                            pos=[PK_UV], leak=0.01),
                           mlp_pairs=2048, mlp_batch=4096, iters=4000, dct_q=[50], shadow_pull=0.01, seed=14,
                           notes="--dct-shadow-pull at its default 0.01 (main.cpp:175)"),
        # 4 x 2048x2048 maps, 1024x1024x4 + 256x256x8 bilinear, 64,64, population 16384, 256K batches
        "material2048": Workload("material2048",
                                 Layout(2048, 2048, [(1024, 1024, 4, False), (256, 256, 8, False)], [64, 64], T=4,
                                        pos=[PK_UV], leak=0.0),
                                 mlp_pairs=8192, mlp_batch=262144, iters=1000, seed=15, textures=4),
    }
