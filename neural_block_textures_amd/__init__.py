"""MI355X (gfx950) backend for the Evolution-Strategies training loop of neural_block_textures.

The product is libntc_hip.so (built from csrc/ by build.py): hand-written HIP kernels behind the
reference's ntc_cuda::Trainer interface (include/ntc_cuda.h) and a C ABI (include/ntc_hip.h).
This package is the Python mirror of that interface (trainer.py) plus the synthetic workload
generator the benchmark and tests use (synth.py).
"""
from .trainer import (DctDesc, Layout, ModelDesc, PK_LV1LOCAL, PK_UV, QesDesc, Trainer, library)

__all__ = ["Trainer", "Layout", "ModelDesc", "QesDesc", "DctDesc", "PK_UV", "PK_LV1LOCAL", "library"]
