"""ctypes binding of the CPU oracle (oracle/libntc_oracle.so) and of the reference build
(oracle/_ref/libntc_ref*.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, never by the product package. Every helper takes numpy arrays and returns numpy arrays.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libntc_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libntc_ref.so")
REF_FAST_SO = os.path.join(HERE, "_ref", "libntc_ref_fast.so")
REF_FAST_V4_SO = os.path.join(HERE, "_ref", "libntc_ref_fast_v4.so")

MAX_LEVELS, MAX_POS, MAX_OUT, MAX_HIDDEN = 3, 16, 12, 8
NS_LAT, NS_MLP, NS_BATCH_PIX, NS_BATCH_TEX = 1, 2, 3, 4


class OrLevel(C.Structure):
    _fields_ = [("W", C.c_int), ("H", C.c_int), ("C", C.c_int), ("nearest", C.c_int), ("off", C.c_longlong)]


class OrModel(C.Structure):
    _fields_ = [("W", C.c_int), ("H", C.c_int), ("nout", C.c_int), ("nlev", C.c_int),
                ("lv", OrLevel * MAX_LEVELS), ("npos", C.c_int), ("pos", C.c_int * MAX_POS),
                ("nin", C.c_int), ("nhidden", C.c_int), ("hidden", C.c_int * MAX_HIDDEN),
                ("leak", C.c_float), ("clamp_out", C.c_int), ("cw", C.c_float * MAX_OUT), ("wsum", C.c_float)]


class OrDct(C.Structure):
    _fields_ = [("C", C.c_int), ("BW", C.c_int), ("BH", C.c_int), ("dc_step", C.c_int), ("deadzone", C.c_int),
                ("lo_w16", C.c_int), ("lam_t16", C.c_float * 16), ("step", C.POINTER(C.c_int)),
                ("code", C.POINTER(C.c_uint8)), ("sym", C.POINTER(C.c_int16))]


class OrTrainCfg(C.Structure):
    _fields_ = [("seed", C.c_uint64), ("mlp_pairs", C.c_int), ("mlp_batch", C.c_int), ("mlp_sigma", C.c_float),
                ("mlp_lr", C.c_float), ("lat_pairs", C.c_int), ("lat_sigma", C.c_float), ("lat_lr", C.c_float),
                ("qat", C.c_int), ("qat_ch", C.c_int * 16), ("fd_from", C.c_int), ("fd_h", C.c_float)]


class OrTrainState(C.Structure):
    _fields_ = [("z", C.POINTER(C.c_float)), ("p", C.POINTER(C.c_float)), ("wm", C.POINTER(C.c_float)),
                ("wv", C.POINTER(C.c_float)), ("wt", C.c_int), ("zm", C.POINTER(C.c_float)),
                ("zv", C.POINTER(C.c_float)), ("zt", C.c_int), ("lat_step_no", C.c_int)]


class OrPrintIn(C.Structure):
    _fields_ = [("qbits", C.c_int), ("qat", C.c_int), ("qat_ch", C.c_int * 16), ("qes_on", C.c_int), ("qes_live", C.c_int),
                ("qes_bits", C.c_int * MAX_LEVELS), ("qes_lo", C.POINTER(C.c_float)), ("qes_range", C.POINTER(C.c_float)),
                ("dct_live", C.c_int), ("dct", C.POINTER(OrDct)), ("dc_raw_bits", C.c_int), ("dct_ctx", C.c_int)]


class OrBitrate(C.Structure):
    _fields_ = [(n, C.c_double) for n in ("bpp_fp32", "bpp_q8", "bpp_q8_ent", "bpp_q8_ctx", "bpp_ctx_level0", "bpp_est",
                                          "bits_mlp", "bits_raw_latent", "bits_header")]


class OrDctStats(C.Structure):
    _fields_ = [("raw", C.c_double * 7), ("h0", C.c_double * 7), ("ctx", C.c_double * 7)] + \
               [(n, C.c_double) for n in ("raw_total", "h0_total", "ctx_total", "code_raw", "code_h0", "code_ctx", "header")] + \
               [(n, C.c_longlong) for n in ("nblk", "ntok_nz", "ntok_eob", "nmag_over")] + \
               [(n, C.c_double) for n in ("nz_mean", "lnz_mean", "eob_only_frac")]


DCT_COUNTS_PER_CH = 65 + 257 + 64 * 65 + 64 * 257 + 64 + 64 + 4097 + 16 + 4096 + 256 + 3
DCT_COUNTS_TAIL = 5


@dataclass
class Model:
    """A decoder layout: image size, latent levels (W, H, C, nearest), positional kinds, MLP."""
    W: int
    H: int
    levels: list            # [(W, H, C, nearest), ...]
    hidden: list
    T: int = 1
    pos: list = field(default_factory=lambda: [0])   # 0 = uv, 1 = lv1local
    leak: float = 0.01
    clamp_out: bool = False
    weights: list = None    # per-texture loss weight

    @property
    def nout(self):
        return 3 * self.T

    @property
    def nin(self):
        return sum(l[2] for l in self.levels) + 2 * len(self.pos)

    def offsets(self):
        off, o = [], 0
        for (w, h, c, _) in self.levels:
            off.append(o)
            o += w * h * c
        return off, o

    @property
    def nz(self):
        return self.offsets()[1]

    @property
    def nparams(self):
        n, cur = 0, self.nin
        for h in self.hidden:
            n += h * cur + h
            cur = h
        return n + self.nout * cur + self.nout

    def cw(self):
        w = self.weights or [1.0] * self.T
        return [float(w[c // 3]) for c in range(self.nout)], float(np.float32(sum(np.float32(x) for x in w)))

    def to_c(self) -> OrModel:
        m = OrModel()
        m.W, m.H, m.nout, m.nlev = self.W, self.H, self.nout, len(self.levels)
        off, _ = self.offsets()
        for l, (w, h, c, nr) in enumerate(self.levels):
            m.lv[l] = OrLevel(w, h, c, int(bool(nr)), off[l])
        m.npos = len(self.pos)
        for q, k in enumerate(self.pos):
            m.pos[q] = k
        m.nin = self.nin
        m.nhidden = len(self.hidden)
        for l, h in enumerate(self.hidden):
            m.hidden[l] = h
        m.leak = self.leak
        m.clamp_out = int(self.clamp_out)
        cw, wsum = self.cw()
        for c in range(self.nout):
            m.cw[c] = cw[c]
        m.wsum = wsum
        return m


def model_of(layout) -> OrModel:
    """OrModel of any layout-like object (W, H, levels, hidden, T, pos, leak, clamp_out, weights)."""
    if isinstance(layout, OrModel):
        return layout
    m = Model(layout.W, layout.H, list(layout.levels), list(layout.hidden), T=layout.T, pos=list(layout.pos),
              leak=layout.leak, clamp_out=layout.clamp_out, weights=layout.weights)
    return m.to_c()


def _f(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _d(a):
    return a.ctypes.data_as(C.POINTER(C.c_double))


def _i(a):
    return a.ctypes.data_as(C.POINTER(C.c_int))


def _load(path):
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built (run `make -C oracle` or __graft_entry__.build())")
    return C.CDLL(path)


_P = C.c_void_p
_SIGS = {
    "mse_of": (None, [_P, _P, C.c_int, C.c_int, C.c_int, _P, C.c_float, C.c_int, C.c_int, _P, _P]),
    "gauss": (C.c_float, [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint64]),
    "noise_u32": (C.c_uint32, [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint64]),
    "noise_uniform": (C.c_uint32, [C.c_uint32, C.c_uint32]),
    "gauss_fill": (None, [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint64, C.c_longlong, _P]),
    "gauss_radius": (C.c_float, [C.c_uint32]),
    "gauss_factors": (None, [C.c_uint32, C.c_longlong, _P, _P]),
    "shadow_pull": (None, [_P, _P, C.c_longlong, C.c_float]),
    "gauss_cosine": (C.c_float, [C.c_uint32]),
    "features": (None, [_P, _P, C.c_int, C.c_int, _P]),
    "mlp_forward": (None, [_P, _P, _P, _P]),
    "decode_full": (None, [_P, _P, _P, _P]),
    "decode_err": (None, [_P, _P, _P, _P, _P]),
    "loss_subset": (C.c_double, [_P, _P, _P, _P, _P, C.c_int]),
    "draw_batch": (None, [C.c_uint64, C.c_int, C.c_int, C.c_int, _P]),
    "mlp_es_eval": (None, [_P, _P, _P, _P, C.c_uint64, C.c_int, C.c_float, C.c_int, _P, C.c_int, _P, _P, _P, _P]),
    "mlp_es_grad": (None, [C.c_longlong, C.c_int, C.c_uint64, C.c_int, C.c_float, _P, _P]),
    "adam": (None, [_P, _P, _P, _P, C.c_longlong, C.c_float, C.c_int]),
    "mlp_fd_eval": (None, [_P, _P, _P, _P, C.c_float, _P, C.c_int, _P, _P, _P]),
    "fd_grad": (None, [C.c_longlong, _P, _P, _P]),
    "lat_grad": (None, [_P, _P, _P, _P, _P, C.c_uint64, C.c_int, C.c_float, C.c_int, C.c_uint, _P, C.c_float,
                        _P, _P, _P, _P]),
    "lat_scatter": (None, [_P, _P, _P, C.c_int, C.c_uint, C.c_float, _P]),
    "qat_grid": (None, [_P]),
    "qat_index": (C.c_int, [C.c_float, C.c_int]),
    "qat_search": (None, [_P, _P, _P, _P, _P, _P]),
    "qes_index": (C.c_int, [C.c_float, C.c_float, C.c_float, C.c_int]),
    "qes_fit": (None, [_P, _P, C.c_int, _P, _P, _P, _P]),
    "qes_snap_level": (C.c_longlong, [_P, C.c_int, _P, _P, _P, _P, _P, _P, C.c_int]),
    "dct_tables": (None, [_P, _P, _P]),
    "dct_build_steps": (None, [C.c_int, C.c_int, _P]),
    "dct_fwd8": (None, [_P, _P]),
    "dct_inv8": (None, [_P, _P]),
    "dct_quant_dc": (C.c_int, [C.c_float, C.c_int]),
    "dct_quant_ac": (C.c_int, [C.c_float, C.c_int, C.c_int, C.c_int, C.c_int]),
    "dct_dequant_ac": (C.c_float, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "dct_block_bits": (C.c_int, [_P, C.c_int]),
    "dct_quantize_block": (C.c_int, [_P, _P, C.c_int, C.c_float, C.c_int, C.c_int, C.c_int, _P, _P, _P]),
    "dct_code_of_gain": (C.c_int, [C.c_double]),
    "dct_snap_level0": (None, [_P, _P, _P, _P, _P, _P]),
    "dct_recon_level0": (None, [_P, _P, _P, _P]),
    "dct_probe_codes": (None, [_P, _P, _P, _P, _P]),
    "dct_rate_pair": (None, [_P, _P, _P, _P, C.c_float, _P]),
    "f32_to_f16": (C.c_uint16, [C.c_float, _P]),
    "f16_to_f32": (C.c_float, [C.c_uint16]),
    "q8_index": (C.c_int, [C.c_float, C.c_float, C.c_float, C.c_int]),
}
_ORACLE_ONLY = {
    "gauss_fill", "gauss_radius", "gauss_cosine", "mlp_es_eval", "mlp_es_grad", "adam", "mlp_fd_eval",
    "fd_grad", "lat_grad", "lat_scatter", "dct_tables", "round_fp16", "train_iter",
}


class Lib:
    """One of the two CPU implementations: prefix 'or_' (the oracle) or 'ref_' (the reference)."""

    def __init__(self, path, prefix):
        self.lib = _load(path)
        self.prefix = prefix
        for name, (res, args) in _SIGS.items():
            fn = getattr(self.lib, prefix + name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
            setattr(self, "_" + name, fn)
        for fn in ("bitrate_stats", "dct_analyze", "latent_stats", "print_counts_size", "print_counts"):
            f = getattr(self.lib, prefix + fn, None)
            if f is not None:
                f.restype = None
                f.argtypes = {"bitrate_stats": [_P, _P, C.c_longlong, _P, _P, _P, _P], "dct_analyze": [_P, C.c_int, C.c_int, _P],
                              "latent_stats": [_P, C.c_int, _P, _P, _P, _P], "print_counts_size": [_P, _P, _P, _P],
                              "print_counts": [_P, _P, _P, _P, _P, _P, _P]}[fn]
        if prefix == "or_":
            self.lib.or_host_isa_level.restype = C.c_int
            self.lib.or_train_iter.restype = C.c_double
            self.lib.or_train_iter.argtypes = [_P, _P, _P, _P, C.c_int, C.c_int]
            self.lib.or_round_fp16.restype = C.c_int
            self.lib.or_round_fp16.argtypes = [_P, C.c_longlong, _P]
            self.lib.or_dct_tables.argtypes = [_P, _P, _P]
        else:
            L = self.lib
            L.ref_mlp_step.restype = C.c_double
            L.ref_mlp_step.argtypes = [_P, _P, _P, _P, C.c_uint64, C.c_int, C.c_float, C.c_float, C.c_int, C.c_int,
                                       _P, _P, _P, _P, _P]
            L.ref_mlp_step_fd.restype = C.c_double
            L.ref_mlp_step_fd.argtypes = [_P, _P, _P, _P, C.c_uint64, C.c_int, C.c_float, C.c_float, C.c_int,
                                          _P, _P, _P, _P, _P]
            L.ref_draw_batch.argtypes = [C.c_uint64, C.c_int, C.c_int, _P, _P]
            L.ref_lat_step.argtypes = [_P, _P, _P, _P, C.c_uint64, C.c_int, C.c_float, C.c_float, C.c_int, C.c_int,
                                       _P, _P, _P, _P]
            L.ref_qat_search.argtypes = [_P, _P, _P, _P, _P]
            L.ref_qat_grid.argtypes = [_P]
            L.ref_dct_tables.argtypes = [_P, _P, _P]
            L.ref_dct_selftest.restype = C.c_int
            L.ref_ntcb_selfcheck.restype = C.c_int
            L.ref_train_create.restype = C.c_void_p
            L.ref_train_create.argtypes = [_P, _P, _P, _P, _P]
            L.ref_train_create_dct.restype = C.c_void_p
            L.ref_train_create_dct.argtypes = [_P, _P, _P, _P, _P, _P, C.c_float, C.c_int, C.c_int]
            L.ref_train_create_dct_sched.restype = C.c_void_p
            L.ref_train_create_dct_sched.argtypes = [_P, _P, _P, _P, _P, _P, C.c_float, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
            L.ref_train_set_shadow_pull.argtypes = [C.c_void_p, C.c_float]
            L.ref_shadow_pull.argtypes = [_P, _P, C.c_longlong, C.c_float]
            L.ref_train_get_zdec.argtypes = [C.c_void_p, _P]
            L.ref_train_round_fp16.restype = C.c_int
            L.ref_train_round_fp16.argtypes = [C.c_void_p]
            L.ref_train_get_dct_codes.argtypes = [C.c_void_p, _P]
            L.ref_train_save.restype = C.c_int
            L.ref_train_save.argtypes = [C.c_void_p, C.c_char_p]
            L.ref_train_load.restype = C.c_int
            L.ref_train_load.argtypes = [C.c_void_p, C.c_char_p]
            L.ref_train_iter.restype = C.c_double
            L.ref_train_iter.argtypes = [C.c_void_p, C.c_int, C.c_int]
            L.ref_train_get.argtypes = [C.c_void_p, _P, _P]
            L.ref_train_destroy.argtypes = [C.c_void_p]
            L.ref_omp_threads.restype = C.c_int

    # ---- noise
    def gauss(self, seed, stream, step, pair, index):
        return self._gauss(seed, stream, step, pair, index)

    def gauss_fill(self, seed, stream, step, pair, index0, n):
        out = np.empty(n, np.float32)
        self._gauss_fill(seed, stream, step, pair, index0, n, out.ctypes.data)
        return out

    # ---- decoder
    def features(self, m, z, px, py):
        mc = model_of(m)
        f = np.zeros(128, np.float32)
        self._features(C.byref(mc), z.ctypes.data, px, py, f.ctypes.data)
        return f[: mc.nin]

    def mlp_forward(self, m, p, x):
        mc = model_of(m)
        out = np.zeros(12, np.float32)
        self._mlp_forward(C.byref(mc), p.ctypes.data, np.ascontiguousarray(x, np.float32).ctypes.data,
                          out.ctypes.data)
        return out[: mc.nout]

    def decode_full(self, m, p, z):
        mc = model_of(m)
        img = np.zeros(mc.W * mc.H * mc.nout, np.float32)
        self._decode_full(C.byref(mc), p.ctypes.data, z.ctypes.data, img.ctypes.data)
        return img

    def decode_err(self, m, p, z, tgt):
        mc = model_of(m)
        err = np.zeros(mc.W * mc.H, np.float32)
        self._decode_err(C.byref(mc), p.ctypes.data, z.ctypes.data, tgt.ctypes.data, err.ctypes.data)
        return err

    def loss_subset(self, m, p, z, tgt, idx):
        idx = np.ascontiguousarray(idx, np.int32)
        return self._loss_subset(C.byref(model_of(m)), p.ctypes.data, z.ctypes.data, tgt.ctypes.data,
                                 idx.ctypes.data, len(idx))

    # ---- oracle-only training pieces (prefix or_)
    def draw_batch(self, seed, it, M, npix):
        idx = np.empty(M, np.int32)
        self._draw_batch(seed, it, M, npix, idx.ctypes.data)
        return idx

    def mlp_es_eval(self, m, p0, z, tgt, seed, it, sigma, N, idx):
        """per pair: dl, lsum, l+, l- (MlpTrainer::step's pair loop)"""
        idx = np.ascontiguousarray(idx, np.int32)
        dl, ls, lp, lm = (np.zeros(N) for _ in range(4))
        self._mlp_es_eval(C.byref(model_of(m)), p0.ctypes.data, z.ctypes.data, tgt.ctypes.data, seed, it, sigma, N,
                          idx.ctypes.data, len(idx), dl.ctypes.data, ls.ctypes.data, lp.ctypes.data, lm.ctypes.data)
        return dl, ls, lp, lm

    def mlp_es_grad(self, P, N, seed, it, sigma, dl):
        g = np.zeros(P, np.float32)
        dl = np.ascontiguousarray(dl, np.float64)
        self._mlp_es_grad(P, N, seed, it, sigma, dl.ctypes.data, g.ctypes.data)
        return g

    def adam(self, theta, g, m, v, lr, t):
        """in place on theta, m, v (float32 arrays)"""
        self._adam(theta.ctypes.data, np.ascontiguousarray(g, np.float32).ctypes.data, m.ctypes.data, v.ctypes.data,
                   theta.size, lr, t)

    def mlp_fd_eval(self, m, p0, z, tgt, h, idx):
        idx = np.ascontiguousarray(idx, np.int32)
        P = p0.size
        dl, hh = np.zeros(P), np.zeros(P)
        l0 = C.c_double()
        self._mlp_fd_eval(C.byref(model_of(m)), p0.ctypes.data, z.ctypes.data, tgt.ctypes.data, h, idx.ctypes.data,
                          len(idx), dl.ctypes.data, hh.ctypes.data, C.addressof(l0))
        return dl, hh, l0.value

    def fd_grad(self, dl, hh):
        g = np.zeros(dl.size, np.float32)
        self._fd_grad(dl.size, np.ascontiguousarray(dl).ctypes.data, np.ascontiguousarray(hh).ctypes.data,
                      g.ctypes.data)
        return g

    def lat_grad(self, m, p, zdec, zshadow, tgt, seed, step_no, sigma, K, mask, dct=None, rate_scale=0.0,
                 want_dpix=False):
        mc = model_of(m)
        nz = sum(mc.lv[l].W * mc.lv[l].H * mc.lv[l].C for l in range(mc.nlev))
        g = np.zeros(nz, np.float32)
        dpix = np.zeros(K * mc.W * mc.H, np.float32) if want_dpix else None
        nbc = dct.BW * dct.BH * dct.C if dct is not None else 0
        dbits = np.zeros(max(nbc, 1), np.int32)
        hits = C.c_int()
        self._lat_grad(C.byref(mc), p.ctypes.data, zdec.ctypes.data, zshadow.ctypes.data, tgt.ctypes.data, seed,
                       step_no, sigma, K, mask, C.byref(dct) if dct is not None else None, rate_scale, g.ctypes.data,
                       dpix.ctypes.data if dpix is not None else None, dbits.ctypes.data, C.addressof(hits))
        return g, dpix, dbits[:nbc], hits.value

    def lat_scatter(self, m, eps, dpix, K, mask, sigma):
        """the latent gradient of K pairs from given dpix [K][W*H] and eps [K][nz] (or_lat_grad's scatter)"""
        mc = model_of(m)
        nz = sum(mc.lv[l].W * mc.lv[l].H * mc.lv[l].C for l in range(mc.nlev))
        g = np.zeros(nz, np.float32)
        e, d = np.ascontiguousarray(eps, np.float32), np.ascontiguousarray(dpix, np.float32)
        assert e.size == K * nz and d.size == K * mc.W * mc.H
        self._lat_scatter(C.byref(mc), e.ctypes.data, d.ctypes.data, K, mask, sigma, g.ctypes.data)
        return g

    def qat_search(self, m, p, z, tgt, ch_bits, grid):
        """in place on level 0 of z"""
        bits = np.zeros(16, np.int32)
        bits[: len(ch_bits)] = ch_bits
        self._qat_search(C.byref(model_of(m)), p.ctypes.data, z.ctypes.data, tgt.ctypes.data, bits.ctypes.data,
                         np.ascontiguousarray(grid, np.float32).ctypes.data)


    # ---- the progress print's statistics (bitrate_stats, dct_analyze, latent_stats; the histograms behind them)
    def bitrate_stats(self, m, pin, P, z, zdec):
        """(OrBitrate, the quantized latent zq)"""
        mc = model_of(m)
        out, zq = OrBitrate(), np.zeros(z.size, np.float32)
        getattr(self.lib, self.prefix + "bitrate_stats")(C.byref(mc), C.byref(pin), int(P), z.ctypes.data, zdec.ctypes.data,
                                                          C.byref(out), zq.ctypes.data)
        return out, zq

    def dct_analyze(self, d, dc_raw_bits, ctx):
        out = OrDctStats()
        getattr(self.lib, self.prefix + "dct_analyze")(C.byref(d), dc_raw_bits, int(ctx), C.byref(out))
        return out

    def latent_stats(self, m, level, z):
        a, b, c = C.c_float(), C.c_float(), C.c_float()
        getattr(self.lib, self.prefix + "latent_stats")(C.byref(model_of(m)), level, z.ctypes.data, C.byref(a), C.byref(b),
                                                         C.byref(c))
        return a.value, b.value, c.value

    def print_counts(self, m, pin, z, zdec):
        """(bitrate histograms, lohi [3][64][2], dct histograms) in the layout ntc_oracle.h documents"""
        mc = model_of(m)
        nb, nd = C.c_longlong(), C.c_longlong()
        self.lib.or_print_counts_size(C.byref(mc), C.byref(pin), C.byref(nb), C.byref(nd))
        hb, lohi, hd = np.zeros(max(nb.value, 1), np.int64), np.zeros(3 * 64 * 2, np.float32), np.zeros(max(nd.value, 1), np.int64)
        self.lib.or_print_counts(C.byref(mc), C.byref(pin), z.ctypes.data, zdec.ctypes.data, hb.ctypes.data, lohi.ctypes.data,
                                 hd.ctypes.data)
        return hb[: nb.value], lohi, hd[: nd.value]


def print_in(qbits=8, qat_ch=None, qes_bits=None, qes_on=False, qes_live=False, qes_lo=None, qes_range=None, dct=None,
             dc_raw_bits=8, dct_ctx=False):
    """an OrPrintIn (the arrays it points at are kept alive on the returned object)"""
    pin = OrPrintIn()
    pin.qbits = qbits
    if qat_ch:
        pin.qat = max(qat_ch)
        for c, b in enumerate(qat_ch):
            pin.qat_ch[c] = b
    pin.qes_on, pin.qes_live = int(qes_on), int(qes_live)
    for l, b in enumerate(qes_bits or []):
        pin.qes_bits[l] = b
    lo = np.zeros(3 * 64, np.float32) if qes_lo is None else np.ascontiguousarray(qes_lo, np.float32)
    rg = np.ones(3 * 64, np.float32) if qes_range is None else np.ascontiguousarray(qes_range, np.float32)
    pin.qes_lo, pin.qes_range = _f(lo), _f(rg)
    pin._keep = (lo, rg, dct)
    if dct is not None:
        pin.dct_live, pin.dct, pin.dc_raw_bits = 1, C.pointer(dct), dc_raw_bits
    pin.dct_ctx = int(dct_ctx)
    return pin


def oracle() -> Lib:
    return Lib(ORACLE_SO, "or_")


def host_isa() -> str:
    """the widest x86-64 level the host CPU and OS support, by cpuid (or_host_isa_level): "x86-64-v4" with
    AVX-512 F/BW/CD/DQ/VL, "x86-64-v3" with AVX2/FMA/BMI2, else "x86-64" """
    return {4: "x86-64-v4", 3: "x86-64-v3"}.get(oracle().lib.or_host_isa_level(), "x86-64")


def reference_path(fast: bool = False, isa: str = "x86-64-v3") -> str:
    """the reference build for an ISA level; "auto" = the widest one built that the host supports"""
    if not fast:
        return REF_SO
    if isa == "auto":
        isa = host_isa()
        if isa == "x86-64-v4" and not os.path.exists(REF_FAST_V4_SO):
            isa = "x86-64-v3"
    return REF_FAST_V4_SO if isa == "x86-64-v4" else REF_FAST_SO


def reference(fast: bool = False, isa: str = "x86-64-v3") -> Lib:
    return Lib(reference_path(fast, isa), "ref_")


def have_reference(fast: bool = False) -> bool:
    return os.path.exists(REF_FAST_SO if fast else REF_SO)
