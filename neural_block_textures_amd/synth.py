"""Seeded synthetic inputs for the benchmark and the parity tests.

The reference trains on PNG files; its synthetic fallback was removed. The workloads here follow
the benchmark's recipe: an RGB8 texture is 4 octaves of value noise plus random axis-aligned hard
edges and a smooth colour gradient in [0, 255]; a 4-map material (albedo, normal, roughness, AO
like) is derived from one seeded height field. Targets are u8 / 255.0f as the reference's PNG
loader converts them (main.cpp:319), interleaved per pixel [r0 g0 b0 r1 g1 b1 ...] (main.cpp:298-300).
The latent starts N(0, lat_init) and the MLP with He-scaled normals and zero biases
(main.cpp:586-599, 3539-3541); --qat snaps level 0 to its grid (main.cpp:2067-2071).
"""
from __future__ import annotations

import numpy as np


def _value_noise(rng, W, H, cells):
    g = rng.random((cells + 1, cells + 1)).astype(np.float64)
    y = np.linspace(0, cells, H, endpoint=False) + 0.5 * cells / H
    x = np.linspace(0, cells, W, endpoint=False) + 0.5 * cells / W
    yi, xi = np.floor(y).astype(int), np.floor(x).astype(int)
    fy, fx = y - yi, x - xi
    sy, sx = fy * fy * (3 - 2 * fy), fx * fx * (3 - 2 * fx)
    a = g[yi][:, xi]
    b = g[yi][:, xi + 1]
    c = g[yi + 1][:, xi]
    d = g[yi + 1][:, xi + 1]
    top = a + (b - a) * sx[None, :]
    bot = c + (d - c) * sx[None, :]
    return top + (bot - top) * sy[:, None]


def height_field(seed: int, W: int, H: int) -> np.ndarray:
    """4 octaves of value noise in [0, 1]."""
    rng = np.random.default_rng(seed)
    h = np.zeros((H, W))
    amp, tot = 1.0, 0.0
    for o in range(4):
        h += amp * _value_noise(rng, W, H, 4 << o)
        tot += amp
        amp *= 0.5
    return h / tot


def rgb_texture(seed: int, W: int, H: int) -> np.ndarray:
    """H x W x 3 uint8: value-noise octaves + axis-aligned hard edges + a smooth colour gradient."""
    rng = np.random.default_rng(seed + 1000003)
    out = np.empty((H, W, 3))
    gy, gx = np.meshgrid(np.linspace(0, 1, H), np.linspace(0, 1, W), indexing="ij")
    for c in range(3):
        n = height_field(seed * 7 + c, W, H)
        a, b = rng.uniform(-0.5, 0.5, 2)
        out[..., c] = 0.55 * n + 0.3 * (0.5 + a * (gx - 0.5) + b * (gy - 0.5))
    for _ in range(6):   # hard edges: axis-aligned rectangles of a flat colour offset
        x0, x1 = np.sort(rng.integers(0, W, 2))
        y0, y1 = np.sort(rng.integers(0, H, 2))
        out[y0:y1 + 1, x0:x1 + 1, :] += rng.uniform(-0.25, 0.25, 3)
    return np.clip(np.rint(out * 255.0), 0, 255).astype(np.uint8)


def material(seed: int, W: int, H: int) -> list:
    """Four H x W x 3 uint8 maps derived from one height field: albedo, normal, roughness, AO."""
    h = height_field(seed, W, H)
    rng = np.random.default_rng(seed + 17)
    tint = rng.uniform(0.3, 1.0, 3)
    albedo = np.clip(h[..., None] * tint[None, None, :] + 0.1 * rgb_texture(seed, W, H) / 255.0, 0, 1)
    dy, dx = np.gradient(h * 8.0)
    nrm = np.stack([-dx, -dy, np.ones_like(h)], -1)
    nrm /= np.linalg.norm(nrm, axis=-1, keepdims=True)
    normal = 0.5 * nrm + 0.5
    rough = np.repeat(np.clip(1.0 - 0.8 * h + 0.1 * np.sin(20 * h), 0, 1)[..., None], 3, -1)
    k = 7
    pad = np.pad(h, k, mode="edge")
    blur = np.zeros_like(h)
    for oy in range(-k, k + 1, 2):
        for ox in range(-k, k + 1, 2):
            blur += pad[k + oy:k + oy + H, k + ox:k + ox + W]
    blur /= ((2 * k) // 2 + 1) ** 2
    ao = np.repeat(np.clip(1.0 - 2.0 * np.maximum(blur - h, 0.0), 0, 1)[..., None], 3, -1)
    return [np.clip(np.rint(m * 255.0), 0, 255).astype(np.uint8) for m in (albedo, normal, rough, ao)]


def target_from_maps(maps: list) -> np.ndarray:
    """W*H*3T float32 target, each value u8 / 255.0f, textures interleaved per pixel."""
    H, W, _ = maps[0].shape
    t = np.concatenate([m.astype(np.float32) for m in maps], axis=-1) / np.float32(255.0)
    return np.ascontiguousarray(t.reshape(W * H * 3 * len(maps)), dtype=np.float32)


def qat_grid() -> np.ndarray:
    """QAT_GRID[9][257] (main.cpp:2054-2057): -1 + (2k) / levels in float."""
    g = np.zeros((9, 257), np.float32)
    for b in range(1, 9):
        levels = np.float32((1 << b) - 1)
        k = np.arange(1 << b, dtype=np.float32)
        g[b, : 1 << b] = np.float32(-1.0) + (np.float32(2.0) * k) / levels
    return g


def qat_snap(v: np.ndarray, bits: int, grid: np.ndarray) -> np.ndarray:
    """qat_snap (main.cpp:2060-2065): lround((v + 1) * 0.5 * levels), clamped, looked up."""
    levels = (1 << bits) - 1
    x = ((v.astype(np.float32) + np.float32(1.0)) * np.float32(0.5) * np.float32(levels)).astype(np.float64)
    k = np.clip(np.floor(np.abs(x) + 0.5) * np.sign(x), 0, levels).astype(np.int64)   # half away from zero, exact in double
    return grid[bits][k]


def init_model(layout, seed: int, lat_init: float = 0.1, qat_bits=None):
    """(z, p): latent N(0, lat_init), He-init weights with zero biases, --qat level 0 snapped."""
    rng = np.random.default_rng(seed)
    z = (rng.standard_normal(layout.nz) * lat_init).astype(np.float32)
    widths = [layout.nin] + list(layout.hidden) + [layout.nout]
    p = np.zeros(layout.nparams, np.float32)
    o = 0
    for l in range(1, len(widths)):
        last = l + 1 == len(widths)
        s = np.sqrt((1.0 if last else 2.0) / widths[l - 1])
        n = widths[l] * widths[l - 1]
        p[o:o + n] = (rng.standard_normal(n) * s).astype(np.float32)
        o += n + widths[l]
    if qat_bits:
        g = qat_grid()
        C0 = layout.levels[0][2]
        n0 = layout.levels[0][0] * layout.levels[0][1] * C0
        lv0 = z[:n0].reshape(-1, C0)
        for c in range(C0):
            lv0[:, c] = qat_snap(lv0[:, c], qat_bits[c], g)
        z[:n0] = lv0.reshape(-1)
    return z, p
