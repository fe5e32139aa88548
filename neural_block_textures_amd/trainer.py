"""Python mirror of ntc_cuda::Trainer over the C ABI of libntc_hip.so (include/ntc_hip.h).

Method names, argument meaning and error behaviour follow the reference's cuda/ntc_cuda.h:78-132:
``init`` raises ``ValueError`` with the backend's reason for a model outside the envelope (the
reference returns false plus a reason), every other misuse ends the process as the reference's
backend does. Host buffers are numpy arrays; every call that reads or fills one is synchronous.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libntc_hip.so")

MAX_LEVELS, MAX_POS, MAX_OUT, MAX_HIDDEN, MAX_CH, MAX_QES_CH, MAX_DCT_CH = 3, 16, 12, 8, 16, 64, 4
PK_UV, PK_LV1LOCAL = 0, 1


class LevelDesc(C.Structure):
    _fields_ = [("W", C.c_int), ("H", C.c_int), ("C", C.c_int), ("off", C.c_size_t), ("nearest", C.c_bool)]


class PosDesc(C.Structure):
    _fields_ = [("kind", C.c_int)]


class ModelDesc(C.Structure):
    _fields_ = [
        ("W", C.c_int), ("H", C.c_int), ("T", C.c_int), ("nlev", C.c_int), ("lv", LevelDesc * MAX_LEVELS),
        ("npos", C.c_int), ("pos", PosDesc * MAX_POS), ("nin", C.c_int), ("nout", C.c_int), ("nhidden", C.c_int),
        ("hidden", C.c_int * MAX_HIDDEN), ("leak", C.c_float), ("clamp_out", C.c_bool), ("cw", C.c_float * MAX_OUT),
        ("wsum", C.c_float), ("qat_bits", C.c_int * MAX_CH), ("qat", C.c_int), ("qat_grid", C.POINTER(C.c_float)),
        ("qes_bits", C.c_int * MAX_LEVELS), ("dct", C.c_int), ("dct_C", C.c_int), ("dct_N", C.c_int),
        ("dct_dc_step", C.c_int), ("dct_q", C.c_int * MAX_DCT_CH), ("dct_basis", C.POINTER(C.c_float)),
        ("dct_zigzag", C.POINTER(C.c_int)), ("max_pairs", C.c_int), ("max_batch", C.c_int), ("seed", C.c_uint64),
    ]


class QesDesc(C.Structure):
    _fields_ = [
        ("bits", C.c_int * MAX_LEVELS), ("live", C.c_int), ("frozen", C.c_int),
        ("lo", (C.c_float * MAX_QES_CH) * MAX_LEVELS), ("hi", (C.c_float * MAX_QES_CH) * MAX_LEVELS),
        ("range", (C.c_float * MAX_QES_CH) * MAX_LEVELS), ("grid_off", (C.c_int * MAX_QES_CH) * MAX_LEVELS),
    ]


class DctDesc(C.Structure):
    _fields_ = [
        ("live", C.c_int), ("C", C.c_int), ("BW", C.c_int), ("BH", C.c_int), ("N", C.c_int), ("dc_step", C.c_int),
        ("rate_es", C.c_int), ("rate_trunc", C.c_int), ("rate_scale", C.c_float), ("lam_t16", C.c_float * 16),
        ("lo_w16", C.c_int), ("deadzone", C.c_int),
    ]


_lib = None


class PrintStats(C.Structure):
    """ntc_print_stats: the progress line's figures (bitrate_stats, the quantized latent's error, latent_stats,
    dct_analyze)"""
    _fields_ = [(n, C.c_double) for n in ("bpp_fp32", "bpp_q8", "bpp_q8_ent", "bpp_q8_ctx", "bpp_ctx_level0", "bpp_est",
                                          "bits_mlp", "bits_raw_latent", "bits_header")] + \
               [("q_tex_mse", C.c_double * 4), ("q_weighted_mse", C.c_double), ("lat_mean", C.c_float * MAX_LEVELS),
                ("lat_sd", C.c_float * MAX_LEVELS), ("lat_max", C.c_float * MAX_LEVELS), ("dct_live", C.c_int),
                ("dct_raw", C.c_double * 7), ("dct_h0", C.c_double * 7), ("dct_ctx", C.c_double * 7),
                ("dct_raw_total", C.c_double), ("dct_h0_total", C.c_double), ("dct_ctx_total", C.c_double),
                ("dct_nblk", C.c_longlong), ("dct_ntok_nz", C.c_longlong), ("dct_ntok_eob", C.c_longlong),
                ("dct_nmag_over", C.c_longlong), ("dct_nz_mean", C.c_double), ("dct_lnz_mean", C.c_double),
                ("dct_eob_only_frac", C.c_double)]


def library() -> C.CDLL:
    """The HIP backend. Raises if it is not built: there is no fallback path."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m neural_block_textures_amd.build` "
                               "(or __graft_entry__.build()) first")
        lib = C.CDLL(LIB_PATH)
        P = C.c_void_p
        sig = {
            "ntc_trainer_create": (P, []),
            "ntc_trainer_destroy": (None, [P]),
            "ntc_trainer_init": (C.c_int, [P, C.POINTER(ModelDesc), P, P, P, C.c_char_p, C.c_size_t]),
            "ntc_trainer_banner": (C.c_size_t, [P, C.c_char_p, C.c_size_t]),
            "ntc_trainer_upload_model": (None, [P, P, P]),
            "ntc_trainer_download_model": (None, [P, P, P]),
            "ntc_trainer_set_qes": (None, [P, C.POINTER(QesDesc), P, C.c_size_t]),
            "ntc_trainer_snap_latent": (None, [P]),
            "ntc_trainer_shadow_pull": (None, [P, C.c_size_t, C.c_size_t, C.c_float]),
            "ntc_trainer_download_zq": (None, [P, P]),
            "ntc_trainer_set_dct": (None, [P, C.POINTER(DctDesc), P, P, P]),
            "ntc_trainer_download_dct": (None, [P, P, P]),
            "ntc_trainer_download_dct_rate": (None, [P, P, P, P, P, P, P]),
            "ntc_trainer_mlp_step": (None, [P, C.c_int, C.c_float, C.c_float, C.c_int, C.c_int]),
            "ntc_trainer_mlp_step_fd": (None, [P, C.c_int, C.c_float, C.c_float, C.c_int]),
            "ntc_trainer_reset_mlp_adam": (None, [P]),
            "ntc_trainer_mlp_stats": (None, [P, P, P]),
            "ntc_trainer_lat_step": (None, [P, C.c_int, C.c_float, C.c_float, C.c_int]),
            "ntc_trainer_qat_search": (None, [P]),
            "ntc_trainer_decode_full": (None, [P, P, P]),
            "ntc_trainer_debug_last_batch": (C.c_size_t, [P, P, C.c_size_t]),
            "ntc_trainer_debug_last_dl": (C.c_size_t, [P, P, C.c_size_t]),
            "ntc_trainer_debug_last_zgrad": (C.c_size_t, [P, P, C.c_size_t]),
            "ntc_abi_sizeof": (C.c_size_t, [C.c_char_p]),
            "ntc_trainer_debug_last_losses": (C.c_size_t, [P, P, P, C.c_size_t]),
            "ntc_trainer_debug_last_wgrad": (C.c_size_t, [P, P, C.c_size_t]),
            "ntc_trainer_debug_last_dpix": (C.c_size_t, [P, P, C.c_size_t]),
            "ntc_trainer_nparams": (C.c_longlong, [P]),
            "ntc_trainer_nz": (C.c_longlong, [P]),
            "ntc_trainer_stream": (P, [P]),
            "ntc_trainer_synchronize": (None, [P]),
            "ntc_trainer_set_profiling": (None, [P, C.c_int]),
            "ntc_trainer_set_profiling_only": (None, [P, C.c_char_p]),
            "ntc_trainer_kernel_time": (C.c_int, [P, C.c_char_p, P, P]),
            "ntc_trainer_on_matrix_cores": (C.c_int, [P, C.c_char_p]),
            "ntc_trainer_set_matrix_cores": (None, [P, C.c_int]),
            "ntc_trainer_set_lat_group": (None, [P, C.c_int]),
            "ntc_trainer_set_profiling_every": (None, [P, C.c_int]),
            "ntc_jit_compile_check": (C.c_int, [C.POINTER(ModelDesc), C.c_char_p, C.POINTER(C.c_double), C.c_char_p, C.c_size_t]),
            "ntc_trainer_dct_probe": (None, [P, P, P]),
            "ntc_trainer_dct_refit": (None, [P, P]),
            "ntc_trainer_decode_error": (None, [P, P, C.c_int, C.c_int, P, P]),
            "ntc_trainer_decode_error_noalloc": (None, [P, P, C.c_int, C.c_int, P, P]),
            "ntc_trainer_print_stats": (None, [P, C.c_int, C.c_int, C.c_int, C.POINTER(PrintStats)]),
            "ntc_trainer_debug_print_counts": (C.c_size_t, [P, P, C.c_size_t, P, P, C.c_size_t, P]),
            "ntc_trainer_decode_rgb8": (None, [P, P]),
            "ntc_trainer_debug_gauss": (None, [P, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint64, C.c_size_t, P]),
            "ntc_trainer_debug_noise_factors": (None, [P, C.c_uint32, C.c_size_t, P, P]),
            "ntc_trainer_debug_copy_calibration": (None, [P, C.c_size_t, C.c_int]),
            "ntc_debug_device_allocations": (None, [P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


def _f32(a, n=None):
    a = np.ascontiguousarray(a, dtype=np.float32)
    if n is not None and a.size != n:
        raise ValueError(f"expected {n} floats, got {a.size}")
    return a


@dataclass
class Layout:
    """A decoder layout in the reference's terms: image size, textures, latent levels
    (W, H, C, nearest), positional kinds, hidden widths, leak, output mode, loss weights."""
    W: int
    H: int
    levels: list
    hidden: list
    T: int = 1
    pos: list = field(default_factory=lambda: [PK_UV])
    leak: float = 0.01
    clamp_out: bool = False
    weights: list = None

    @property
    def nout(self):
        return 3 * self.T

    @property
    def nin(self):
        return sum(l[2] for l in self.levels) + 2 * len(self.pos)

    @property
    def offsets(self):
        off, o = [], 0
        for (w, h, c, _) in self.levels:
            off.append(o)
            o += w * h * c
        return off

    @property
    def nz(self):
        return sum(w * h * c for (w, h, c, _) in self.levels)

    @property
    def nparams(self):
        n, cur = 0, self.nin
        for h in self.hidden:
            n += h * cur + h
            cur = h
        return n + self.nout * cur + self.nout

    def loss_weights(self):
        w = self.weights or [1.0] * self.T
        cw = [float(w[c // 3]) for c in range(self.nout)]
        ws = np.float32(0.0)
        for x in w:
            ws = np.float32(ws + np.float32(x))
        return cw, float(ws)


class Trainer:
    """ntc_cuda::Trainer (cuda/ntc_cuda.h:78-132) on one MI355X."""

    def __init__(self):
        self._lib = library()
        self._h = self._lib.ntc_trainer_create()
        self._keep = []
        self.layout = None

    def close(self):
        if getattr(self, "_h", None):
            self._lib.ntc_trainer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- init
    @staticmethod
    def model_desc(layout: Layout, *, max_pairs=64, max_batch=4096, seed=1, qat_bits=None, qat_grid=None,
                   qes_bits=None, dct=None, dct_basis=None, dct_zigzag=None) -> ModelDesc:
        d = ModelDesc()
        d.W, d.H, d.T = layout.W, layout.H, layout.T
        d.nlev = len(layout.levels)
        for l, (off, (w, h, c, nr)) in enumerate(zip(layout.offsets, layout.levels)):
            d.lv[l] = LevelDesc(w, h, c, off, bool(nr))
        d.npos = len(layout.pos)
        for q, k in enumerate(layout.pos):
            d.pos[q].kind = k
        d.nin, d.nout = layout.nin, layout.nout
        d.nhidden = len(layout.hidden)
        for l, h in enumerate(layout.hidden):
            d.hidden[l] = h
        d.leak = layout.leak
        d.clamp_out = layout.clamp_out
        cw, wsum = layout.loss_weights()
        for c in range(MAX_OUT):
            d.cw[c] = cw[c] if c < layout.nout else 0.0
        d.wsum = wsum
        if qat_bits:
            for c, b in enumerate(qat_bits):
                d.qat_bits[c] = b
            d.qat = max(qat_bits)
            d.qat_grid = qat_grid.ctypes.data_as(C.POINTER(C.c_float))
        for l, b in enumerate(qes_bits or []):
            d.qes_bits[l] = b
        if dct:
            d.dct, d.dct_C, d.dct_N, d.dct_dc_step = 1, dct["C"], 8, dct.get("dc_step", 4)
            for c, q in enumerate(dct.get("q", [50] * dct["C"])):
                d.dct_q[c] = q
            d.dct_basis = dct_basis.ctypes.data_as(C.POINTER(C.c_float))
            d.dct_zigzag = dct_zigzag.ctypes.data_as(C.POINTER(C.c_int))
        d.max_pairs, d.max_batch, d.seed = max_pairs, max_batch, seed
        return d

    def init(self, d: ModelDesc, z, p, target, layout: Layout | None = None):
        """Trainer::init. Raises ValueError(reason) where the reference returns false."""
        self.layout = layout
        z = np.ascontiguousarray(z, np.float32)
        p = np.ascontiguousarray(p, np.float32)
        target = np.ascontiguousarray(target, np.float32)
        why = C.create_string_buffer(512)
        ok = self._lib.ntc_trainer_init(self._h, C.byref(d), z.ctypes.data, p.ctypes.data, target.ctypes.data, why, 512)
        if not ok:
            raise ValueError(why.value.decode())
        self.nz = int(self._lib.ntc_trainer_nz(self._h))
        self.P = int(self._lib.ntc_trainer_nparams(self._h))
        self.W, self.H, self.nout = d.W, d.H, d.nout
        self.dct_n = (d.W // 8) * (d.H // 8) * d.dct_C if d.dct else 0
        return self

    def banner(self) -> str:
        buf = C.create_string_buffer(512)
        self._lib.ntc_trainer_banner(self._h, buf, 512)
        return buf.value.decode()

    # ---- model transfer and snapping
    def upload_model(self, z, p):
        z, p = _f32(z, self.nz), _f32(p, self.P)
        self._lib.ntc_trainer_upload_model(self._h, z.ctypes.data, p.ctypes.data)

    def download_model(self):
        z = np.empty(self.nz, np.float32)
        p = np.empty(self.P, np.float32)
        self._lib.ntc_trainer_download_model(self._h, z.ctypes.data, p.ctypes.data)
        return z, p

    def set_qes(self, q: QesDesc, grid):
        grid = _f32(grid)
        self._lib.ntc_trainer_set_qes(self._h, C.byref(q), grid.ctypes.data, grid.size)

    def snap_latent(self):
        self._lib.ntc_trainer_snap_latent(self._h)

    def shadow_pull(self, off, n, f):
        self._lib.ntc_trainer_shadow_pull(self._h, off, n, f)

    def download_zq(self):
        zq = np.empty(self.nz, np.float32)
        self._lib.ntc_trainer_download_zq(self._h, zq.ctypes.data)
        return zq

    def set_dct(self, d: DctDesc, code, sym, step):
        code = np.ascontiguousarray(code, np.uint8)
        sym = np.ascontiguousarray(sym, np.int16)
        step = np.ascontiguousarray(step, np.int32)
        self._lib.ntc_trainer_set_dct(self._h, C.byref(d), code.ctypes.data, sym.ctypes.data, step.ctypes.data)

    def download_dct(self):
        sym = np.empty(self.dct_n * 64, np.int16)
        code = np.empty(self.dct_n, np.uint8)
        self._lib.ntc_trainer_download_dct(self._h, sym.ctypes.data, code.ctypes.data)
        return sym, code

    def download_dct_rate(self):
        bits = np.empty(self.dct_n, np.int32)
        dbits = np.empty(self.dct_n, np.int32)
        v = [C.c_int() for _ in range(4)]
        self._lib.ntc_trainer_download_dct_rate(self._h, bits.ctypes.data, dbits.ctypes.data,
                                                *[C.addressof(x) for x in v])
        return bits, dbits, v[0].value, v[1].value, v[2].value, v[3].value

    def dct_probe(self):
        """the device's decoder sensitivity probe: (codes uint8 [block][channel], block gains float32)"""
        code = np.empty(self.dct_n, np.uint8)
        gain = np.empty(self.dct_n, np.float32)
        self._lib.ntc_trainer_dct_probe(self._h, code.ctypes.data, gain.ctypes.data)
        return code, gain

    def dct_refit(self):
        """probe on the device, replace the codes, re-snap level 0; returns the new codes"""
        code = np.empty(self.dct_n, np.uint8)
        self._lib.ntc_trainer_dct_refit(self._h, code.ctypes.data)
        return code

    def decode_rgb8(self):
        """the decode rounded to 8 bits (save_png's rounding): uint8 [H*W*nout]"""
        out = np.empty(self.layout.W * self.layout.H * self.layout.nout, np.uint8)
        self._lib.ntc_trainer_decode_rgb8(self._h, out.ctypes.data)
        return out

    def decode_error(self, ew=0, eh=0, z=None):
        """mse_of of the device's decode (of its decode buffer, or of the host latent z):
        (per-texture 8-bit MSE, weighted MSE)"""
        T = max(1, self.layout.nout // 3) if self.layout else 4
        tex = np.zeros(4, np.float64)
        wt = C.c_double()
        zh = None if z is None else _f32(z, self.nz)
        self._lib.ntc_trainer_decode_error(self._h, _ptr(zh), ew, eh, tex.ctypes.data, C.addressof(wt))
        return tex[:T], wt.value

    def decode_error_noalloc(self, ew=0, eh=0, z=None):
        """decode_error with no device allocation at call time (its partial sums in the library's static
        per-GPU scratch; at most 2^24 pixels in the extent)"""
        T = max(1, self.layout.nout // 3) if self.layout else 4
        tex = np.zeros(4, np.float64)
        wt = C.c_double()
        zh = None if z is None else _f32(z, self.nz)
        self._lib.ntc_trainer_decode_error_noalloc(self._h, _ptr(zh), ew, eh, tex.ctypes.data, C.addressof(wt))
        return tex[:T], wt.value

    def print_stats(self, qbits=8, ew=0, eh=0) -> PrintStats:
        """the reference's progress-line figures from the device (bitrate_stats as a progress print runs it, the
        quantized latent's 8-bit error, latent_stats, dct_analyze of a live --dct-q plane); no model download"""
        out = PrintStats()
        self._lib.ntc_trainer_print_stats(self._h, qbits, ew, eh, C.byref(out))
        return out

    def debug_print_counts(self):
        """(bitrate histograms, lohi [3 x 64 x 2], dct histograms) of the last print_stats"""
        nd = C.c_size_t()
        nb = self._lib.ntc_trainer_debug_print_counts(self._h, None, 0, None, None, 0, C.byref(nd))
        hb, lohi, hd = np.zeros(max(nb, 1), np.int64), np.zeros(3 * 64 * 2, np.float32), np.zeros(max(nd.value, 1), np.int64)
        self._lib.ntc_trainer_debug_print_counts(self._h, hb.ctypes.data, nb, lohi.ctypes.data, hd.ctypes.data, nd.value, None)
        return hb[:nb], lohi, hd[:nd.value]

    # ---- steps
    def mlp_step(self, it, sigma, lr, N, M):
        self._lib.ntc_trainer_mlp_step(self._h, it, sigma, lr, N, M)

    def mlp_step_fd(self, it, h, lr, M):
        self._lib.ntc_trainer_mlp_step_fd(self._h, it, h, lr, M)

    def reset_mlp_adam(self):
        self._lib.ntc_trainer_reset_mlp_adam(self._h)

    def mlp_stats(self):
        a, b = C.c_double(), C.c_double()
        self._lib.ntc_trainer_mlp_stats(self._h, C.addressof(a), C.addressof(b))
        return a.value, b.value

    def lat_step(self, it, sigma, lr, K):
        self._lib.ntc_trainer_lat_step(self._h, it, sigma, lr, K)

    def qat_search(self):
        self._lib.ntc_trainer_qat_search(self._h)

    def decode_full(self, z_host=None):
        img = np.empty(self.W * self.H * self.nout, np.float32)
        zh = None if z_host is None else _f32(z_host, self.nz)
        self._lib.ntc_trainer_decode_full(self._h, _ptr(zh), img.ctypes.data)
        return img

    # ---- verification helpers
    def debug_last_batch(self):
        n = self._lib.ntc_trainer_debug_last_batch(self._h, None, 0)
        out = np.empty(n, np.int32)
        self._lib.ntc_trainer_debug_last_batch(self._h, out.ctypes.data, n)
        return out

    def debug_last_dl(self):
        n = self._lib.ntc_trainer_debug_last_dl(self._h, None, 0)
        out = np.empty(n, np.float64)
        self._lib.ntc_trainer_debug_last_dl(self._h, out.ctypes.data, n)
        return out

    def debug_last_losses(self):
        """(l+, l-) per pair of the last MLP step (per weight for a central-difference step)"""
        n = self._lib.ntc_trainer_debug_last_losses(self._h, None, None, 0)
        lp, lm = np.empty(n), np.empty(n)
        self._lib.ntc_trainer_debug_last_losses(self._h, lp.ctypes.data, lm.ctypes.data, n)
        return lp, lm

    def debug_last_wgrad(self):
        out = np.empty(self.P, np.float32)
        self._lib.ntc_trainer_debug_last_wgrad(self._h, out.ctypes.data, self.P)
        return out

    def debug_last_zgrad(self):
        out = np.empty(self.nz, np.float32)
        self._lib.ntc_trainer_debug_last_zgrad(self._h, out.ctypes.data, self.nz)
        return out

    def debug_last_dpix(self):
        """the per-pixel loss differences of the last latent step, [K, W*H]"""
        n = self._lib.ntc_trainer_debug_last_dpix(self._h, None, 0)
        out = np.empty(n, np.float32)
        self._lib.ntc_trainer_debug_last_dpix(self._h, out.ctypes.data, n)
        return out.reshape(-1, self.layout.W * self.layout.H) if n else out

    def debug_gauss(self, stream, step, pair, index0, n):
        out = np.empty(n, np.float32)
        self._lib.ntc_trainer_debug_gauss(self._h, stream, step, pair, index0, n, out.ctypes.data)
        return out

    def debug_noise_factors(self, k0, n):
        rad = np.empty(n, np.float32)
        cosv = np.empty(n, np.float32)
        self._lib.ntc_trainer_debug_noise_factors(self._h, k0, n, rad.ctypes.data, cosv.ctypes.data)
        return rad, cosv

    # ---- instrumentation
    @staticmethod
    def device_allocations():
        """(hipMalloc calls, hipFree calls) the library has made in this process"""
        a, f = C.c_longlong(), C.c_longlong()
        library().ntc_debug_device_allocations(C.byref(a), C.byref(f))
        return a.value, f.value

    def debug_copy_calibration(self, n, reps=1):
        self._lib.ntc_trainer_debug_copy_calibration(self._h, n, reps)

    def synchronize(self):
        self._lib.ntc_trainer_synchronize(self._h)

    def set_profiling(self, on: bool, only=None, every: int = 1):
        """HIP events around every launch (of the kernel families in `only`, if given; one launch in `every` of each)"""
        self._lib.ntc_trainer_set_profiling_only(self._h, ",".join(only).encode() if only else b"")
        self._lib.ntc_trainer_set_profiling_every(self._h, int(every))
        self._lib.ntc_trainer_set_profiling(self._h, 1 if on else 0)

    def on_matrix_cores(self, stage: str) -> bool:
        """whether the stage ("pop_eval", "lat_pair", "qat_search") runs on the FP32 matrix cores; "pop_pair": whether ES
        steps take a kernel that shares a pair's first layer, "pop_pair_own": whether that is k_pop_pair_own"""
        return bool(self._lib.ntc_trainer_on_matrix_cores(self._h, stage.encode()))

    def set_matrix_cores(self, on: bool):
        """on=False: every stage on the VALU kernels from the next call on (instrumentation)"""
        self._lib.ntc_trainer_set_matrix_cores(self._h, 1 if on else 0)

    def set_lat_group(self, pairs: int):
        """latent steps in groups of at most `pairs` pairs (0: by the 1 GiB buffer budget); the same results"""
        self._lib.ntc_trainer_set_lat_group(self._h, int(pairs))

    @staticmethod
    def jit_compile_check(d: ModelDesc, arch: str = "gfx950"):
        """compile (hipRTC, no device) the kernels a trainer specialises at init for d's shape:
        (seconds, "") or (None, the compiler's reason)"""
        sec, why = C.c_double(), C.create_string_buffer(4096)
        ok = library().ntc_jit_compile_check(C.byref(d), arch.encode(), C.byref(sec), why, 4096)
        return (sec.value, "") if ok else (None, why.value.decode(errors="replace"))

    def kernel_time(self, name):
        ms, n = C.c_double(), C.c_longlong()
        self._lib.ntc_trainer_kernel_time(self._h, name.encode(), C.addressof(ms), C.addressof(n))
        return ms.value, n.value
