// The figures of the reference's progress line without downloading the model (main.cpp:4155-4212, where
// --cuda downloads the latent and the weights at every print and computes them on the host):
//   bitrate_stats (main.cpp:2273-2352) as a progress print runs it (main.cpp:4171: the order-0 figure stands
//     in for the (up, left) context estimate), and the quantized latent it returns, decoded and scored
//     (mse_of, main.cpp:4172-4174);
//   latent_stats of every level of the shadow (main.cpp:2211-2216);
//   dct_analyze of a live --dct-q level 0 (main.cpp:1080-1208) with the code grid's context estimate, as the
//     progress line's token group calls it (main.cpp:4180).
// Every one of those figures is a sum over integer histograms (per level and channel: the quantization
// indices, and the DPCM residuals of levels >= 1; per DCT channel: run, magnitude, their contexts, DC
// residuals, codes and the code grid's (up, left) contexts). The kernels fill the histograms exactly (integer
// atomics: the same counts in any order); the host turns them into the figures with the reference's own
// loops over bins. Bitrate figures are then the reference's bit for bit; dct_analyze's per-class sums are
// the same terms added per histogram bin instead of per token (within 1e-13 relative).
#include <math.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "trainer_impl.hpp"

namespace ntc_hip {

// ---------------------------------------------------------------- histogram layout (the oracle's or_print_counts layout)
constexpr int kDctPerCh = 65 + 257 + 64 * 65 + 64 * 257 + 64 + 64 + 4097 + 16 + 4096 + 256 + 3;
constexpr int kDctTail = 5;
enum : int { kDRun = 0, kDMag = 65, kDCtxRun = 322, kDCtxMag = 322 + 4160, kDCtxR = 4482 + 16448, kDCtxM = 20930 + 64,
             kDDcRes = 20994 + 64, kDCode = 21058 + 4097, kDTri = 25155 + 16, kDPair = 25171 + 4096, kDScal = 25267 + 4256 };
static_assert(kDScal + 3 == kDctPerCh, "the per-channel DCT histogram layout");

// one (level, channel) of the bitrate histograms
struct StatSeg {
    int l, c, C, W, H, kind, bits;   // kind 0: continuous (post-hoc grid), 1: discrete --qat level 0, 2: live --qes
    int hoff, roff;                  // index bins, residual bins (-1: level 0 has none)
    long long off;                   // the level's first value
};
constexpr int kMaxSegs = 3 * 64;
struct StatSegs { int n; StatSeg s[kMaxSegs]; };

// a float as an unsigned key that orders like the float (for integer min / max atomics)
__device__ __forceinline__ unsigned fkey(float f) {
    const unsigned u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__host__ __device__ inline float fkey_inv(unsigned k) {
    const unsigned u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// Per level: each block's sum and sum of squares of the values in double (the thread's own, then a fixed tree),
// the largest magnitude, and - for the level's continuous channels - each channel's least and greatest value.
__global__ void __launch_bounds__(256) k_level_reduce(const float* __restrict__ z, long long off, int ntex, int C, int want_range,
                                                     double* __restrict__ part, unsigned* __restrict__ maxabs,
                                                     unsigned* __restrict__ keys) {
    __shared__ unsigned lo_s[64], hi_s[64];
    __shared__ double red[2][4];
    for (int c = threadIdx.x; c < C; c += 256) { lo_s[c] = 0xFFFFFFFFu; hi_s[c] = 0u; }
    __syncthreads();
    double s = 0.0, s2 = 0.0;
    unsigned mx = 0u;
    for (int t = blockIdx.x * 256 + threadIdx.x; t < ntex; t += gridDim.x * 256) {
        const float* v = z + off + (long long)t * C;
        for (int c = 0; c < C; c++) {
            const float x = v[c];
            s += (double)x;
            s2 += (double)x * (double)x;
            mx = max(mx, __float_as_uint(fabsf(x)));
            if (want_range) { atomicMin(&lo_s[c], fkey(x)); atomicMax(&hi_s[c], fkey(x)); }
        }
    }
    s = wave_sum(s); s2 = wave_sum(s2);
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, (unsigned)__shfl_xor((int)mx, o, 64));
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) { red[0][w] = s; red[1][w] = s2; atomicMax(maxabs, mx); }
    __syncthreads();
    if (threadIdx.x == 0) {
        part[2 * blockIdx.x] = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
        part[2 * blockIdx.x + 1] = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    }
    if (want_range)
        for (int c = threadIdx.x; c < C; c += 256) { atomicMin(&keys[2 * c], lo_s[c]); atomicMax(&keys[2 * c + 1], hi_s[c]); }
}

// The quantization index of value i of segment g (bitrate_stats' three kinds, main.cpp:2306-2313) and its value.
__device__ __forceinline__ int seg_index(const StatSeg& g, const ntc_cuda::QesDesc* qes, const unsigned* keys, const float* z,
                                         const float* zdec, long long i, float* q) {
    const int levels = (1 << g.bits) - 1;
    const float x = z[i];
    if (g.kind == 1) { *q = x; return qat_index(x, g.bits); }
    if (g.kind == 2) { *q = zdec[i]; return qes_index(x, qes->lo[g.l][g.c], qes->range[g.l][g.c], levels); }
    const float lo = fkey_inv(keys[(g.l * 64 + g.c) * 2]), hi = fkey_inv(keys[(g.l * 64 + g.c) * 2 + 1]);
    const float range = fmaxf(__fsub_rn(hi, lo), 1e-6f);
    const int k = q8_index(x, lo, range, levels);
    *q = q8_value(k, lo, range, levels);
    return k;
}

// Index and DPCM-residual histograms of every segment (blockIdx.y) over its texels (blockIdx.x chunks), in LDS
// first, and the quantized latent zq (main.cpp:2306-2313). The residual's predictor is floor((left + up) / 2),
// left alone on the first row, up alone on the first column, 0 at the origin (main.cpp:2333-2338).
constexpr int kHistChunk = 2048;
__global__ void __launch_bounds__(256) k_level_hist(StatSegs segs, const ntc_cuda::QesDesc* __restrict__ qes, const unsigned* __restrict__ keys,
                                                   const float* __restrict__ z, const float* __restrict__ zdec, float* __restrict__ zq,
                                                   unsigned* __restrict__ hist) {
    __shared__ unsigned h_s[2 * 4096];
    const StatSeg g = segs.s[blockIdx.y];
    const int nbin = 1 << g.bits, ntex = g.W * g.H;
    const bool resid = g.roff >= 0;
    for (int k = threadIdx.x; k < 2 * nbin; k += 256) h_s[k] = 0u;
    __syncthreads();
    const int t0 = blockIdx.x * kHistChunk, t1 = min(ntex, t0 + kHistChunk);
    for (int t = t0 + (int)threadIdx.x; t < t1; t += 256) {
        const long long i = g.off + (long long)t * g.C + g.c;
        float q;
        const int k = seg_index(g, qes, keys, z, zdec, i, &q);
        zq[i] = q;
        atomicAdd(&h_s[k], 1u);
        if (resid) {
            const int x = t % g.W, y = t / g.W;
            float dummy;
            const int lf = x ? seg_index(g, qes, keys, z, zdec, i - g.C, &dummy) : -1;
            const int up = y ? seg_index(g, qes, keys, z, zdec, i - (long long)g.W * g.C, &dummy) : -1;
            const int pred = (lf >= 0 && up >= 0) ? (lf + up) / 2 : (lf >= 0 ? lf : (up >= 0 ? up : 0));
            atomicAdd(&h_s[nbin + ((k - pred) & (nbin - 1))], 1u);
        }
    }
    __syncthreads();
    for (int k = threadIdx.x; k < nbin; k += 256) {
        if (h_s[k]) atomicAdd(&hist[g.hoff + k], h_s[k]);
        if (resid && h_s[nbin + k]) atomicAdd(&hist[g.roff + k], h_s[nbin + k]);
    }
}

// dct_analyze's first pass (main.cpp:1093-1126) and its code-grid counts (main.cpp:1162-1165, context_entropy_bits
// main.cpp:2242-2258) for one (block, channel) per thread: tokens in zigzag order, every count one integer atomic.
__global__ void __launch_bounds__(256) k_dct_hist(DevDct D, const int16_t* __restrict__ sym, const uint8_t* __restrict__ code,
                                                 unsigned* __restrict__ h) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= D.n) return;
    const int b = i / D.C, c = i - b * D.C;
    const int bx = b % D.BW, by = b / D.BW;
    unsigned* hc = h + (size_t)c * kDctPerCh;
    unsigned* tail = h + (size_t)D.C * kDctPerCh;
    const int16_t* s = sym + (size_t)i * 64;
    const int pred = bx > 0 ? sym[(size_t)(i - D.C) * 64] : (by > 0 ? sym[(size_t)(i - D.BW * D.C) * 64] : 0);
    atomicAdd(&hc[kDDcRes + clampi(s[0] - pred + 2048, 0, 4096)], 1u);
    int run = 0, prev = 0, nz = 0, lnz = 0;
    unsigned over = 0;
    for (int p = 1; p < 64; p++) {
        const int q = s[D.zigzag[p]];
        if (q == 0) { run++; continue; }
        const int aq = abs(q), mag = min(256, aq);
        over += aq > 256;
        atomicAdd(&hc[kDRun + run], 1u); atomicAdd(&hc[kDMag + mag], 1u);
        atomicAdd(&hc[kDCtxRun + prev * 65 + run], 1u); atomicAdd(&hc[kDCtxMag + prev * 257 + mag], 1u);
        atomicAdd(&hc[kDCtxR + prev], 1u); atomicAdd(&hc[kDCtxM + prev], 1u);
        nz++; lnz = p; prev = p; run = 0;
    }
    if (lnz < 63) {
        atomicAdd(&hc[kDRun + 64], 1u); atomicAdd(&hc[kDCtxRun + prev * 65 + 64], 1u); atomicAdd(&hc[kDCtxR + prev], 1u);
        atomicAdd(&hc[kDScal + 1], 1u);
    }
    if (nz) { atomicAdd(&hc[kDScal + 0], (unsigned)nz); atomicAdd(&hc[kDScal + 2], (unsigned)nz); }
    atomicAdd(&tail[0], (unsigned)nz);
    if (nz) { atomicAdd(&tail[1], (unsigned)lnz); atomicAdd(&tail[2], 1u); } else atomicAdd(&tail[3], 1u);
    if (over) atomicAdd(&tail[4], over);
    const int k = code[i];
    const int u = by ? code[i - D.BW * D.C] : 0, lf = bx ? code[i - D.C] : 0;
    atomicAdd(&hc[kDCode + k], 1u); atomicAdd(&hc[kDTri + u * 256 + lf * 16 + k], 1u); atomicAdd(&hc[kDPair + u * 16 + lf], 1u);
}

namespace {

template <class T>
void ensure(T** p, size_t& cap, size_t need) {
    if (need <= cap) return;
    if (*p) (void)ntc_hip::ntc_free(*p);
    NTC_CHECK(ntc_hip::ntc_malloc((void**)p, need * sizeof(T)));
    cap = need;
}

double cl0(double cnt, double tot) { return cnt != 0.0 && tot != 0.0 ? -std::log2(cnt / tot) : 0.0; }   // main.cpp:1130
// -sum_b h[b] log2(h[b] / n), bins ascending (main.cpp:2316-2317)
double h0_of(const long long* h, int nbin, double n) {
    double s = 0.0;
    for (int v = 0; v < nbin; v++)
        if (h[v]) s -= (double)h[v] * std::log2((double)h[v] / n);
    return s;
}

// dct_analyze's per-class bits from the histograms (main.cpp:1128-1170): the terms of the per-token sums, one
// histogram bin at a time
void dct_figures(const std::vector<long long>& hd, int C, size_t nb, int dc_raw_bits, bool ctx_code, ntc_print_stats& o, double* h0_total,
                 double* ctx_total, double* raw_total, double* header) {
    double raw[7] = { 0 }, h0[7] = { 0 }, cx[7] = { 0 };
    for (int c = 0; c < C; c++) {
        const long long* a = hd.data() + (size_t)c * kDctPerCh;
        const long long nrun = a[kDScal + 0], neob = a[kDScal + 1], nsign = a[kDScal + 2];
        const double nrt = (double)(nrun + neob), dnb = (double)nb;
        raw[0] += (double)dc_raw_bits * dnb; raw[1] += 7.0 * (double)nrun; raw[2] += 8.0 * (double)nrun; raw[3] += (double)nrun;
        raw[4] += 7.0 * (double)neob;
        for (int k = 0; k <= 4096; k++) if (a[kDDcRes + k]) { const double t = (double)a[kDDcRes + k] * cl0((double)a[kDDcRes + k], dnb); h0[0] += t; cx[0] += t; }
        for (int r = 0; r < 64; r++) if (a[kDRun + r]) h0[1] += (double)a[kDRun + r] * cl0((double)a[kDRun + r], nrt);
        for (int mg = 0; mg <= 256; mg++) if (a[kDMag + mg]) h0[2] += (double)a[kDMag + mg] * cl0((double)a[kDMag + mg], (double)nrun);
        h0[3] += (double)nsign; cx[3] += (double)nsign;
        if (a[kDRun + 64]) h0[4] += (double)a[kDRun + 64] * cl0((double)a[kDRun + 64], nrt);
        for (int p = 0; p < 64; p++) {
            const double tr = (double)a[kDCtxR + p], tm = (double)a[kDCtxM + p];
            for (int r = 0; r < 64; r++) { const long long v = a[kDCtxRun + p * 65 + r]; if (v) cx[1] += (double)v * cl0((double)v, tr); }
            for (int mg = 0; mg <= 256; mg++) { const long long v = a[kDCtxMag + p * 257 + mg]; if (v) cx[2] += (double)v * cl0((double)v, tm); }
            const long long e = a[kDCtxRun + p * 65 + 64];
            if (e) cx[4] += (double)e * cl0((double)e, tr);
        }
        double ch0 = 0.0;
        for (int k = 0; k < 16; k++) if (a[kDCode + k]) ch0 += (double)a[kDCode + k] * cl0((double)a[kDCode + k], dnb);
        raw[5] += 4.0 * dnb; h0[5] += ch0;
        cx[5] += ctx_code ? h0_of(a + kDTri, 4096, dnb) - h0_of(a + kDPair, 256, dnb) : ch0;
        raw[6] += 96.0; h0[6] += 96.0; cx[6] += 96.0;
    }
    double rt = 0, ht = 0, ct = 0;
    for (int k = 0; k < 7; k++) { rt += raw[k]; ht += h0[k]; ct += cx[k]; }
    if (h0_total) *h0_total = ht;
    if (ctx_total) *ctx_total = ct;
    if (raw_total) *raw_total = rt;
    if (header) *header = raw[6];
    if (ctx_code) {
        for (int k = 0; k < 7; k++) { o.dct_raw[k] = raw[k]; o.dct_h0[k] = h0[k]; o.dct_ctx[k] = cx[k]; }
        o.dct_raw_total = rt; o.dct_h0_total = ht; o.dct_ctx_total = ct;
    }
}

}   // namespace

// The bitrate segments of the model: every (level, channel) except a live DCT level 0, with its kind and bits
// (bitrate_stats main.cpp:2283-2297) and its place in the histogram array.
static int stat_segments(const Impl& I, int qbits, StatSegs& S) {
    memset(&S, 0, sizeof(S));
    int off = 0;
    for (int l = 0; l < I.d.nlev; l++) {
        if (l == 0 && I.dct_live) continue;
        const bool fixed = l == 0 && I.d.qat > 0;
        const bool qes = I.qes && I.qes_h.live && I.qes_h.bits[l] > 0;
        for (int c = 0; c < I.d.lv[l].C; c++) {
            if (S.n >= kMaxSegs) { fprintf(stderr, "ntc_hip backend: print_stats takes at most %d level channels\n", kMaxSegs); exit(1); }
            StatSeg& g = S.s[S.n++];
            g.l = l; g.c = c; g.C = I.d.lv[l].C; g.W = I.d.lv[l].W; g.H = I.d.lv[l].H; g.off = (long long)I.d.lv[l].off;
            g.kind = fixed ? 1 : (qes ? 2 : 0);
            g.bits = fixed ? I.d.qat_bits[c] : (qes ? I.qes_h.bits[l] : ((I.qes && I.d.qes_bits[l] > 0) ? I.d.qes_bits[l] : qbits));
            if (g.bits < 1 || g.bits > 12) { fprintf(stderr, "ntc_hip backend: print_stats: %d-bit level (1 to 12 bits)\n", g.bits); exit(1); }
            g.hoff = off; off += 1 << g.bits;
            g.roff = l >= 1 ? off : -1; if (l >= 1) off += 1 << g.bits;
        }
    }
    return off;
}

void print_stats_impl(Impl& I, int qbits, int ew, int eh, ntc_print_stats* out) {
    if (I.d.nout % 3 != 0) { fprintf(stderr, "ntc_hip backend: print_stats needs RGB textures (nout a multiple of 3)\n"); exit(1); }
    ntc_print_stats o;
    memset(&o, 0, sizeof(o));
    StatSegs S;
    const int nbins = stat_segments(I, qbits, S);
    // ---- latent_stats and the continuous channels' ranges
    const int kRedBlocks = 512;
    ensure(&I.st_part, I.st_part_cap, (size_t)kMaxLevels * kRedBlocks * 2);
    ensure(&I.st_keys, I.st_keys_cap, (size_t)kMaxLevels * 64 * 2 + kMaxLevels);
    std::vector<unsigned> keys0((size_t)kMaxLevels * 64 * 2 + kMaxLevels);
    for (size_t k = 0; k < (size_t)kMaxLevels * 64; k++) { keys0[2 * k] = 0xFFFFFFFFu; keys0[2 * k + 1] = 0u; }
    NTC_CHECK(hipMemcpyAsync(I.st_keys, keys0.data(), keys0.size() * sizeof(unsigned), hipMemcpyHostToDevice, I.stream));
    unsigned* maxabs = I.st_keys + (size_t)kMaxLevels * 64 * 2;
    int nblk[kMaxLevels] = { 0 };
    for (int l = 0; l < I.d.nlev; l++) {
        const int ntex = I.d.lv[l].W * I.d.lv[l].H;
        nblk[l] = std::max(1, std::min(kRedBlocks, (ntex + 255) / 256));
        bool cont = false;
        for (int k = 0; k < S.n; k++) if (S.s[k].l == l && S.s[k].kind == 0) cont = true;
        if (I.d.lv[l].C > 64) { fprintf(stderr, "ntc_hip backend: print_stats takes at most 64 channels per level\n"); exit(1); }
        hipLaunchKernelGGL(k_level_reduce, dim3(nblk[l]), dim3(256), 0, I.stream, I.z, (long long)I.d.lv[l].off, ntex, I.d.lv[l].C,
                           cont ? 1 : 0, I.st_part + (size_t)l * kRedBlocks * 2, maxabs + l, I.st_keys + (size_t)l * 64 * 2);
        NTC_CHECK(hipGetLastError());
    }
    // ---- the index and residual histograms, and the quantized latent
    ensure(&I.st_hist, I.st_hist_cap, (size_t)std::max(nbins, 1));
    ensure(&I.zpost, I.zpost_cap, I.nz);
    NTC_CHECK(hipMemsetAsync(I.st_hist, 0, (size_t)std::max(nbins, 1) * sizeof(unsigned), I.stream));
    if (I.dct_live)   // the DCT-coded plane is the quantized level 0 as it stands
        NTC_CHECK(hipMemcpyAsync(I.zpost, I.zdec, (size_t)I.d.lv[0].W * I.d.lv[0].H * I.d.lv[0].C * sizeof(float), hipMemcpyDeviceToDevice,
                                 I.stream));
    if (S.n) {
        int chunks = 1;
        for (int k = 0; k < S.n; k++) chunks = std::max(chunks, (S.s[k].W * S.s[k].H + kHistChunk - 1) / kHistChunk);
        hipLaunchKernelGGL(k_level_hist, dim3(chunks, S.n), dim3(256), 0, I.stream, S, I.qes ? I.qes_dev : nullptr, I.st_keys, I.z, I.zdec,
                           I.zpost, I.st_hist);
        NTC_CHECK(hipGetLastError());
    }
    // ---- the DCT plane's token histograms
    const int nd = I.dct_live ? I.ddct.C * kDctPerCh + kDctTail : 0;
    if (nd) {
        ensure(&I.st_dct, I.st_dct_cap, (size_t)nd);
        NTC_CHECK(hipMemsetAsync(I.st_dct, 0, (size_t)nd * sizeof(unsigned), I.stream));
        hipLaunchKernelGGL(k_dct_hist, dim3((I.ddct.n + 255) / 256), dim3(256), 0, I.stream, I.ddct, I.dct_sym, I.dct_code, I.st_dct);
        NTC_CHECK(hipGetLastError());
    }
    // ---- download the counts (a few KB to a few hundred KB; never the model)
    std::vector<double> part((size_t)kMaxLevels * kRedBlocks * 2);
    std::vector<unsigned> keys(keys0.size()), hist((size_t)std::max(nbins, 1)), dh((size_t)std::max(nd, 1));
    NTC_CHECK(hipMemcpyAsync(part.data(), I.st_part, part.size() * sizeof(double), hipMemcpyDeviceToHost, I.stream));
    NTC_CHECK(hipMemcpyAsync(keys.data(), I.st_keys, keys.size() * sizeof(unsigned), hipMemcpyDeviceToHost, I.stream));
    if (nbins) NTC_CHECK(hipMemcpyAsync(hist.data(), I.st_hist, (size_t)nbins * sizeof(unsigned), hipMemcpyDeviceToHost, I.stream));
    if (nd) NTC_CHECK(hipMemcpyAsync(dh.data(), I.st_dct, (size_t)nd * sizeof(unsigned), hipMemcpyDeviceToHost, I.stream));
    // ---- the quantized latent's decode and its 8-bit error (mse_of over ew x eh)
    if (ew <= 0 || ew > I.d.W) ew = I.d.W;
    if (eh <= 0 || eh > I.d.H) eh = I.d.H;
    const size_t sblocks = ((size_t)ew * eh + 255) / 256;
    ensure(&I.st_sse, I.st_sse_cap, sblocks * 4);
    launch_decode(I, I.zpost);
    launch_u8_sse(I, ew, eh, I.st_sse);
    std::vector<unsigned long long> sse(sblocks * 4);
    NTC_CHECK(hipMemcpyAsync(sse.data(), I.st_sse, sse.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost, I.stream));
    NTC_CHECK(hipStreamSynchronize(I.stream));
    {
        const int T = I.d.nout / 3;
        const double np = (double)ew * eh;
        double ws = 0.0;
        for (int t = 0; t < T; t++) {
            unsigned long long s = 0;
            for (size_t b = 0; b < sblocks; b++) s += sse[b * 4 + t];
            o.q_tex_mse[t] = (double)s / (3.0 * np);
            ws += (double)I.d.cw[3 * t] * (double)s;
        }
        o.q_weighted_mse = ws / (3.0 * (double)I.d.wsum * np);
    }
    // ---- latent_stats (main.cpp:2211-2216)
    for (int l = 0; l < I.d.nlev; l++) {
        double s = 0.0, s2 = 0.0;
        for (int b = 0; b < nblk[l]; b++) { s += part[((size_t)l * kRedBlocks + b) * 2]; s2 += part[((size_t)l * kRedBlocks + b) * 2 + 1]; }
        const double n = (double)I.d.lv[l].W * I.d.lv[l].H * I.d.lv[l].C;
        o.lat_mean[l] = (float)(s / n);
        o.lat_sd[l] = (float)std::sqrt(std::max(0.0, s2 / n - (s / n) * (s / n)));
        const unsigned mk = keys[(size_t)kMaxLevels * 64 * 2 + l];
        memcpy(&o.lat_max[l], &mk, 4);
    }
    // ---- bitrate_stats (main.cpp:2273-2352)
    I.st_counts.assign(hist.begin(), hist.begin() + nbins);
    I.st_lohi.assign((size_t)kMaxLevels * 64 * 2, 0.0f);
    for (size_t k = 0; k < (size_t)kMaxLevels * 64 * 2; k++) I.st_lohi[k] = fkey_inv(keys[k]);
    I.st_dct_counts.assign(dh.begin(), dh.begin() + nd);
    const double npix = (double)I.d.W * I.d.H;
    o.bits_mlp = (double)I.P * 16.0;
    o.bpp_fp32 = ((double)I.nz * 32.0 + (double)I.P * 32.0) / npix;
    double ent = 0, header = 0, raw = 0, ctx = 0, est = 0;
    const int dc_raw_bits = [&] { int b = 0; const int lv = 512 / std::max(1, I.ddct.dc_step) + 1; while ((1 << b) < lv) b++; return b; }();
    for (int l = 0; l < I.d.nlev; l++) {
        const double ntex = (double)I.d.lv[l].W * I.d.lv[l].H;
        if (l == 0 && I.dct_live) {
            double ht, ct, rt, hd;
            ntc_print_stats dummy;
            dct_figures(I.st_dct_counts, I.ddct.C, (size_t)I.ddct.BW * I.ddct.BH, dc_raw_bits, false, dummy, &ht, &ct, &rt, &hd);
            raw += rt - hd; ent += ht - hd; ctx += ct - hd; est += ht - hd;
            o.bpp_ctx_level0 += (ct - hd) / npix;
            header += hd;
            continue;
        }
        const bool fixed = l == 0 && I.d.qat > 0;
        const bool qes = I.qes && I.qes_h.live && I.qes_h.bits[l] > 0;
        int kind_any = -1, lbits = qbits;
        for (int k = 0; k < S.n; k++) if (S.s[k].l == l) { kind_any = S.s[k].kind; lbits = S.s[k].bits; }
        if (!fixed && !qes) raw += (double)I.d.lv[l].W * I.d.lv[l].H * I.d.lv[l].C * (double)lbits;
        for (int k = 0; k < S.n; k++) {
            const StatSeg& g = S.s[k];
            if (g.l != l) continue;
            const int nb = 1 << g.bits;
            if (fixed || qes) raw += ntex * (double)g.bits;
            std::vector<long long> hv(hist.begin() + g.hoff, hist.begin() + g.hoff + nb);
            const double h = h0_of(hv.data(), nb, ntex);
            ent += h;
            ctx += h;
            if (l == 0) { o.bpp_ctx_level0 += h / npix; est += h; }
            else {
                std::vector<long long> hr(hist.begin() + g.roff, hist.begin() + g.roff + nb);
                est += h0_of(hr.data(), nb, ntex);
            }
        }
        (void)kind_any;
        if (!fixed) header += I.d.lv[l].C * 2 * 32.0;
    }
    o.bpp_q8 = (raw + header + o.bits_mlp) / npix;
    o.bpp_q8_ent = (ent + header + o.bits_mlp) / npix;
    o.bpp_q8_ctx = (ctx + header + o.bits_mlp) / npix;
    o.bpp_est = (est + header + o.bits_mlp) / npix;
    o.bits_raw_latent = raw; o.bits_header = header;
    // ---- dct_analyze with the code grid's context estimate, as the progress line's token group calls it
    if (I.dct_live) {
        const size_t nb = (size_t)I.ddct.BW * I.ddct.BH, nbc = nb * (size_t)I.ddct.C;
        dct_figures(I.st_dct_counts, I.ddct.C, nb, dc_raw_bits, true, o, nullptr, nullptr, nullptr, nullptr);
        const long long* tail = I.st_dct_counts.data() + (size_t)I.ddct.C * kDctPerCh;
        o.dct_live = 1;
        o.dct_nblk = (long long)nb;
        for (int c = 0; c < I.ddct.C; c++) {
            o.dct_ntok_nz += I.st_dct_counts[(size_t)c * kDctPerCh + kDScal + 0];
            o.dct_ntok_eob += I.st_dct_counts[(size_t)c * kDctPerCh + kDScal + 1];
        }
        o.dct_nmag_over = 2 * tail[4];   // dct_analyze counts each |symbol| > 256 in both of its passes (main.cpp:1113, 1147)
        o.dct_nz_mean = (double)tail[0] / (double)nbc;
        o.dct_lnz_mean = tail[2] ? (double)tail[1] / (double)tail[2] : 0.0;
        o.dct_eob_only_frac = (double)tail[3] / (double)nbc;
    }
    *out = o;
}

}   // namespace ntc_hip
