"""Copies a model file the reference ships (out_m1234/model.bin: a 4-texture 512x512 material trained by the
reference, v12 layout) into tests/golden/, with the reference's own decode of it (recon_003000_t*.png of the
same directory, the printed reconstruction at the iteration the model was saved) reduced to two 64x64 crops
per texture and the per-channel sums of the whole image, and the same for recon_q_final_t*.png (the model
with its continuous levels on bitrate_stats' post-hoc 8-bit grid). Run from the repository root where the reference
tree is present:

    python tests/golden/make_model_fixture.py
"""
import os
import shutil

import numpy as np
from PIL import Image

SRC = "/root/reference/out_m1234"
OUT = os.path.dirname(os.path.abspath(__file__))


def main():
    shutil.copyfile(os.path.join(SRC, "model.bin"), os.path.join(OUT, "ref_m1234_model.bin"))
    rgb = np.concatenate([np.asarray(Image.open(os.path.join(SRC, f"recon_003000_t{t}.png")).convert("RGB"))
                          for t in range(4)], axis=2)          # H x W x 12, uint8
    # the same model with its continuous levels on the post-hoc 8-bit grid (recon_q_final_t*.png)
    rq = np.concatenate([np.asarray(Image.open(os.path.join(SRC, f"recon_q_final_t{t}.png")).convert("RGB"))
                         for t in range(4)], axis=2)
    np.savez_compressed(os.path.join(OUT, "ref_m1234_recon.npz"), crop_a=rgb[0:64, 0:64], crop_b=rgb[224:288, 300:364],
                        at_a=np.array([0, 0]), at_b=np.array([224, 300]),
                        channel_sums=rgb.reshape(-1, 12).astype(np.int64).sum(0),
                        q_crop_a=rq[0:64, 0:64], q_crop_b=rq[224:288, 300:364],
                        q_channel_sums=rq.reshape(-1, 12).astype(np.int64).sum(0))
    print("fixture written to", OUT)


if __name__ == "__main__":
    main()
