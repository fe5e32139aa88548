// The shape-templated VALU kernels of the gfx950 ES backend, device code only: compiled into
// libntc_hip.so for the fixed shapes of shapes.hpp, and by hipRTC at init for the shape of a model
// that is none of them (jit.cpp). Their launchers are in kernels_mlp.hip, kernels_latent.hip and
// kernels_quant.hip.
//
// Reference semantics (main.cpp): MlpTrainer::draw_batch 1825-1833, MlpTrainer::step 1836-1876,
// Decoder::decode_full 1712-1718, LatentTrainer::step_impl 1974-2044, qat_search 2088-2139,
// dct_probe_codes 1001-1032.
#pragma once
#include "device_common.hpp"

namespace ntc_hip {

constexpr int kTPB = 256;
constexpr int kTPB_DCT = 64;   // the probe: one (block, channel) per thread

// The Gaussians of an ES step whose population kernel reads them rather than drawing them per chunk (pair i,
// weight k -> eps[i P + k]): blocks first_block and up of the minibatch launch draw them, an independent job
// that would otherwise be a launch of its own. first_block past the grid: none.
struct EpsJob {
    NoiseFix nt;
    uint64_t seed;
    uint32_t step;
    int N, P;
    float* eps;
    int first_block;
};

// The unperturbed first layer of every minibatch slot, for the population kernel that shares it between the members of
// a pair (k_pop_pair): out[u][s] = fl(b_u fb) + sum_i fl(w_ui fb) f_i as one chain of fused multiply-adds in input order
// (the matrix instructions' order), fb the folded activation's scale. w null: none.
struct Lay1Job {
    const float* w;
    float* out;
};

// floats of the first layer's weights and biases (fixed shapes of one hidden width; 1 otherwise)
template <class S, bool = S::kFixed && S::kUniform>
struct FirstLayerSize { static constexpr int value = 1; };
template <class S>
struct FirstLayerSize<S, true> { static constexpr int value = S::kH * (S::kNin + 1); };

// The minibatch (draw_batch with the counter draw): slot s -> pixel, its feature column
// feat[.][s] and target column btgt[.][s] (structure of arrays, so the evaluation reads coalesced).
template <class S>
__global__ void __launch_bounds__(kTPB) k_batch(DevModel m, uint64_t head, int M, int Mcap, const float* __restrict__ zdec,
                                               const float* __restrict__ tgt, int* __restrict__ bidx,
                                               float* __restrict__ feat, float* __restrict__ btgt, EpsJob ej, Lay1Job l1) {
    if ((int)blockIdx.x >= ej.first_block) {
        const long long t = (long long)(blockIdx.x - ej.first_block) * kTPB + threadIdx.x;
        if (t < (long long)ej.N * ej.P) {
            const int i = (int)(t / ej.P), k = (int)(t - (long long)i * ej.P);
            ej.eps[t] = gauss_at(ej.nt, noise_head(ej.seed, NS_MLP, ej.step, (uint32_t)i), (uint64_t)k);
        }
        return;
    }
    // the first layer's weights and biases times fb, once per block (the Lay1Job below reads them from LDS)
    constexpr int kW1 = FirstLayerSize<S>::value;
    __shared__ float w1_s[kW1];
    if constexpr (S::kFixed && S::kUniform) {
        if (l1.w) {   // uniform: the whole block stages, before any thread leaves
            const float fb = 0.5f * (1.0f + m.leak);
            for (int k = (int)threadIdx.x; k < kW1; k += kTPB) w1_s[k] = l1.w[k] * fb;
            __syncthreads();
        }
    }
    const int s = blockIdx.x * kTPB + threadIdx.x;
    if (s >= M) return;
    const uint32_t u = (uint32_t)(noise_bits(head, (uint64_t)s) >> 32);
    const int idx = (int)noise_uniform(u, (uint32_t)m.npix);
    bidx[s] = idx;
    float f[S::kMaxIn];
    features<S>(m, PlainLatent{ zdec }, idx % m.W, idx / m.W, f);
    if constexpr (S::kFixed) {
#pragma unroll
        for (int i = 0; i < S::kNin; i++) feat[(size_t)i * Mcap + s] = f[i];
    } else {
        for (int i = 0; i < m.nin; i++) feat[(size_t)i * Mcap + s] = f[i];
    }
    const float* t = tgt + (size_t)idx * m.nout;
    for (int c = 0; c < m.nout; c++) btgt[(size_t)c * Mcap + s] = t[c];
    if constexpr (S::kFixed && S::kUniform) {
        if (l1.w) {
            constexpr int H = S::kH, NIN = S::kNin;
#pragma unroll
            for (int u = 0; u < H; u++) {
                float a = w1_s[H * NIN + u];
#pragma unroll
                for (int i = 0; i < NIN; i++) a = __builtin_fmaf(w1_s[u * NIN + i], f[i], a);
                l1.out[(size_t)u * Mcap + s] = a;
            }
        }
    }
}

// The population evaluation: block (pair, chunk) evaluates both members of the pair on the
// chunk's minibatch slots; each slot's features are loaded once and run through the two weight
// vectors, whose uniform addresses put the weights in SGPRs. Per-member weighted squared errors
// are summed in double and reduced in a fixed order.
template <class S>
__global__ void __launch_bounds__(kTPB) k_pop_eval(DevModel m, const float* __restrict__ wsets, int M, int Mcap, int chunk,
                                                  int chunks, const float* __restrict__ feat,
                                                  const float* __restrict__ btgt, double* __restrict__ part) {
    __shared__ double red[kTPB / 64];
    const int pair = blockIdx.x, ch = blockIdx.y;
    const float* __restrict__ wp = wsets + (size_t)(2 * pair) * m.P;
    const float* __restrict__ wn = wp + m.P;
    const int s0 = ch * chunk, s1 = min(M, s0 + chunk);
    double ap = 0.0, an = 0.0;
    for (int s = s0 + (int)threadIdx.x; s < s1; s += kTPB) {
        float f[S::kMaxIn], t[S::kMaxOut], o[S::kMaxOut];
        if constexpr (S::kFixed) {
#pragma unroll
            for (int i = 0; i < S::kNin; i++) f[i] = feat[(size_t)i * Mcap + s];
#pragma unroll
            for (int c = 0; c < S::kNout; c++) t[c] = btgt[(size_t)c * Mcap + s];
        } else {
            for (int i = 0; i < m.nin; i++) f[i] = feat[(size_t)i * Mcap + s];
            for (int c = 0; c < m.nout; c++) t[c] = btgt[(size_t)c * Mcap + s];
        }
        mlp_forward<S>(m, wp, f, o);
        ap += pixel_err_d(m, o, t);
        mlp_forward<S>(m, wn, f, o);
        an += pixel_err_d(m, o, t);
    }
    ap = block_sum<kTPB>(ap, red);
    an = block_sum<kTPB>(an, red);
    if (threadIdx.x == 0) {
        part[(size_t)(2 * pair) * chunks + ch] = ap;
        part[(size_t)(2 * pair + 1) * chunks + ch] = an;
    }
}

// Full decode (Decoder::decode_full): one pixel per thread.
template <class S>
__global__ void __launch_bounds__(kTPB) k_decode(DevModel m, const float* __restrict__ w, const float* __restrict__ z,
                                                float* __restrict__ img) {
    const int p = blockIdx.x * kTPB + threadIdx.x;
    if (p >= m.npix) return;
    float f[S::kMaxIn], o[S::kMaxOut];
    features<S>(m, PlainLatent{ z }, p % m.W, p / m.W, f);
    mlp_forward<S>(m, w, f, o);
    float* dst = img + (size_t)p * m.nout;
    for (int c = 0; c < m.nout; c++) dst[c] = o[c];
}

// One antithetic latent pair per blockIdx.y: the pixel's features are built from the decode
// buffer with the pair's texels perturbed by +sg eps and by -sg eps (each texel value one fused
// operation, as the reference perturbs the flat latent before sampling), two MLP forwards, and
// dpix = (e+ - e-) * inv_px with the per-pixel errors fused in float (decode_err).
template <class S>
__global__ void __launch_bounds__(kTPB) k_lat_pair(DevModel m, const float* __restrict__ w, const float* __restrict__ zdec,
                                                  const float* __restrict__ eps, const float* __restrict__ tgt, float sg,
                                                  unsigned mask, float* __restrict__ dpix) {
    const int p = blockIdx.x * kTPB + threadIdx.x;
    if (p >= m.npix) return;
    const int k = blockIdx.y;
    const float* e = eps + (size_t)k * m.nz;
    const int px = p % m.W, py = p / m.W;
    const float* t = tgt + (size_t)p * m.nout;
    float f[S::kMaxIn], o[S::kMaxOut];
    features<S>(m, PerturbedLatent{ zdec, e, sg, mask }, px, py, f);
    mlp_forward<S>(m, w, f, o);
    const float ep = pixel_err_f(m, o, t);
    features<S>(m, PerturbedLatent{ zdec, e, -sg, mask }, px, py, f);
    mlp_forward<S>(m, w, f, o);
    const float em = pixel_err_f(m, o, t);
    dpix[(size_t)k * m.npix + p] = (ep - em) * m.inv_px;
}

// Exact per-texel search on the discrete nearest level 0 (qat_search): one thread per texel;
// channels in order, the current grid value first, then every other value with strict <; the
// cell loss is the double sum over the cell's pixels in raster order. The winner is written to
// the decode buffer at once, so the next channel's features see it. Texels own disjoint cells, so
// threads never read each other's level-0 values.
template <class S>
__global__ void __launch_bounds__(kTPB) k_qat_search(DevModel m, const float* __restrict__ w, float* __restrict__ zdec,
                                                    const float* __restrict__ tgt, const int* __restrict__ ranges,
                                                    const int* __restrict__ qat_bits, const float* __restrict__ grid) {
    const DevLevel& L = m.lv[0];
    const int t = blockIdx.x * kTPB + threadIdx.x;
    if (t >= L.W * L.H) return;
    const int tx = t % L.W, ty = t / L.W;
    const int* R = ranges + L.rng;
    const int x0 = R[tx], x1 = R[L.W + tx], y0 = R[2 * L.W + ty], y1 = R[2 * L.W + L.H + ty];
    if (x0 >= x1 || y0 >= y1) return;
    float* zt = zdec + L.off + (size_t)t * L.C;
    constexpr int CMAX = S::kFixed ? S::kC0 : 16;
#pragma unroll
    for (int c = 0; c < CMAX; c++) {
        if (c >= L.C) continue;
        const int bits = qat_bits[c], levels = (1 << bits) - 1;
        const float* g = grid + bits * 257;
        auto cell_loss = [&](float val) {
            double sum = 0.0;
            for (int py = y0; py < y1; py++)
                for (int px = x0; px < x1; px++) {
                    float f[S::kMaxIn], o[S::kMaxOut];
                    features<S>(m, PlainLatent{ zdec }, px, py, f);
                    f[c] = val;
                    mlp_forward<S>(m, w, f, o);
                    sum += pixel_err_d(m, o, tgt + ((size_t)py * m.W + px) * m.nout);
                }
            return sum;
        };
        int best_k = qat_index(zt[c], bits);
        double best = cell_loss(g[best_k]);
        for (int k = 0; k <= levels; k++) {
            if (k == best_k) continue;
            const double sk = cell_loss(g[k]);
            if (sk < best) { best = sk; best_k = k; }
        }
        zt[c] = g[best_k];
    }
}

// The decoder sensitivity probe of a DCT-coded level 0 (dct_probe_codes, main.cpp:1001-1032), on the
// device: one thread per (block, channel). At the 4 positions (8 bx + {2, 5}, 8 by + {2, 5}) the
// features are built once from the decode buffer and the MLP evaluated with level-0 channel c set to
// -1, -0.5, 0, 0.5, 1; segment gain g = (255 / 16) sqrt(sum_o cw_o (out_{j+1} - out_j)^2 / wsum), block
// gain = RMS over the 16 (position, segment) pairs, code = round(log2(g / g_floor) / 0.6) in [0, 15].
// The reference calls the probe an estimate (not strict FP): the device's expf and log2 can move a
// gain that sits on a code boundary to the neighbouring code.
template <class S>
__global__ void __launch_bounds__(kTPB_DCT) k_dct_probe(DevModel m, const float* __restrict__ w, const float* __restrict__ zdec,
                                                       int BW, int BH, int C, uint8_t* __restrict__ code, float* __restrict__ gain) {
    const int t = blockIdx.x * kTPB_DCT + threadIdx.x;
    if (t >= BW * BH * C) return;
    const int c = t % C, b = t / C, bx = b % BW, by = b / BW;
    const int P[2] = { 2, 5 };
    const float SJ[5] = { -1.0f, -0.5f, 0.0f, 0.5f, 1.0f };
    double acc = 0.0;
    for (int py = 0; py < 2; py++)
        for (int px = 0; px < 2; px++) {
            float f[S::kMaxIn], out[5][S::kMaxOut];
            features<S>(m, PlainLatent{ zdec }, bx * 8 + P[px], by * 8 + P[py], f);
            for (int j = 0; j < 5; j++) {
                f[c] = SJ[j];
                mlp_forward<S>(m, w, f, out[j]);
            }
            for (int j = 0; j < 4; j++) {
                double ss = 0.0;
                for (int o = 0; o < m.nout; o++) {
                    const double d = (double)out[j + 1][o] - (double)out[j][o];
                    ss = __dadd_rn(ss, __dmul_rn(__dmul_rn((double)m.cw[o], d), d));
                }
                const double g = (255.0 / 16.0) * sqrt(ss / (double)m.wsum);
                acc += g * g;
            }
        }
    const double gb = sqrt(acc / 16.0);
    const double gf = 14.0 / 64.0;
    const double gc = gb > gf ? gb : gf;
    const long long k = (long long)round(log2(gc / gf) / 0.6);
    code[t] = (uint8_t)(k < 0 ? 0 : (k > 15 ? 15 : k));
    if (gain) gain[t] = (float)gb;
}

}   // namespace ntc_hip
