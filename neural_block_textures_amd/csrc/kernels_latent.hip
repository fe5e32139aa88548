// Latent-side kernels of the gfx950 ES backend: the latent Gaussians of one step, the antithetic
// pair evaluation over the full image, the footprint gather that turns per-pixel loss differences
// into the latent gradient, and the exhaustive --qat selector search.
//
// Reference semantics (main.cpp): LatentTrainer::step_impl 1974-2044 (perturb texels, decode_err
// twice, raster-order scatter into the distinct taps, grad += w * eps), dct_rate_pass 1935-1952,
// qat_search 2088-2139.
#include "kern_valu.hpp"
#include "jit.hpp"
#include "shapes.hpp"
#include "trainer_impl.hpp"

namespace ntc_hip {


__device__ __forceinline__ int level_of(const DevModel& m, long long i) {
    int l = 0;
    for (int q = 1; q < m.nlev; q++) if (i >= m.lv[q].off) l = q;
    return l;
}

// eps[k][i] = gauss(seed, NS_LAT, step, k0 + k, i) for the ES-perturbed levels (the other levels' entries are
// never read and are left as they are): the group of pairs k0 .. k0 + gridDim.y - 1 of a latent step; the
// first group's pair-0 threads also clear the latent gradient. Grid: latent entries x pairs (blockIdx.y = k).
__global__ void __launch_bounds__(kTPB) k_lat_eps(NoiseFix nt, DevModel m, uint64_t seed, uint32_t step, unsigned mask, int k0,
                                                 float* __restrict__ eps, float* __restrict__ zgrad) {
    const long long i = (long long)blockIdx.x * kTPB + threadIdx.x;
    if (i >= m.nz) return;
    const int k = blockIdx.y;
    if (k0 + k == 0) zgrad[i] = 0.0f;
    const int l = level_of(m, i);
    if ((mask >> l) & 1u) eps[(size_t)k * m.nz + i] = gauss_at(nt, noise_head(seed, NS_LAT, step, (uint32_t)(k0 + k)), (uint64_t)i);
}

// Footprint gather per level (the gather form of the reference's raster-order scatter,
// main.cpp:2011-2037): the loss difference a texel's taps collect from pair k is the sum of dpix[k]
// over the pixel rectangle that reads the texel, in raster order (the rectangle comes from the host's
// range table, built with the same tap arithmetic); then grad += (d * scale) * eps per channel, pair
// after pair. With the --dct-lambda rate term, level 0 also receives (rate_scale * dbits) * scale * eps
// right after each pair's mse term. Block = 16 texels x 4 pairs: the 64 threads sum the footprints
// of four pairs at once (each sum in raster order), then apply the four pairs in order to the texels'
// channels (four threads per texel, each on every fourth channel). A texel's gradient is then final
// (one block owns it), so with `adam` the block also takes the texel's Adam step (the latent ES step's
// update, main.cpp:2036-2037), and with zq_copy writes the new value to the decode copy too (a level that is neither
// --qes nor DCT coded, where the snap would copy it). With `first` the gradient starts from zero rather than from grad
// (the step's first group of pairs).
//
// Blocks past the gather's own (blockIdx.x >= gblocks) draw the next latent step's Gaussians for the perturbed
// levels (the entries lo .. hi - 1 whose level is in `mask`; block d = pair d / eb, entries lo + 128 (d % eb) ..):
// the values k_lat_eps would draw for step next_step, written to eps_next. They run beside the gather's blocks,
// which leave most of the chip idle, so the next step needs no draw launch of its own.
//
// One launch gathers every perturbed level of the step (GatherLevels: blocks start[i] .. start[i + 1] - 1 take level
// lv[i]); the rate term goes to level 0, and zq_copy[i] (or null) is level lv[i]'s decode copy.
constexpr int kGatherTex = 16, kGatherPairs = 4, kGatherRun = 32, kAheadPerBlock = 128;
struct LatAhead {
    NoiseFix nt; uint64_t seed; uint32_t next_step; unsigned mask;
    float* eps_next; int eb; long long lo, hi;
};
struct GatherLevels {
    int n;
    int lv[kMaxLevels];
    int start[kMaxLevels + 1];
    float* zq_copy[kMaxLevels];
};
__global__ void __launch_bounds__(kGatherTex * kGatherPairs) k_lat_gather(DevModel m, GatherLevels G, int K, float scale,
                                                                         const float* __restrict__ dpix,
                                                                         const float* __restrict__ eps, const int* __restrict__ ranges,
                                                                         int rate0, float rate_scale, int dct_bw, int dct_n,
                                                                         const int32_t* __restrict__ dbits, float* __restrict__ grad,
                                                                         int first, int adam, float* __restrict__ z, float* __restrict__ zm,
                                                                         float* __restrict__ zv, float lr, float c1, float c2, LatAhead ah) {
    if ((int)blockIdx.x >= G.start[G.n]) {   // a draw-ahead block (uniform: the whole block returns here)
        const int d = (int)blockIdx.x - G.start[G.n], k = d / ah.eb;
        const uint64_t head = noise_head(ah.seed, NS_LAT, ah.next_step, (uint32_t)k);
        const long long i0 = ah.lo + (long long)(d - k * ah.eb) * kAheadPerBlock, i1 = min(ah.hi, i0 + kAheadPerBlock);
        for (long long i = i0 + threadIdx.x; i < i1; i += kGatherTex * kGatherPairs)
            if ((ah.mask >> level_of(m, i)) & 1u) ah.eps_next[(size_t)k * m.nz + i] = gauss_at(ah.nt, head, (uint64_t)i);
        return;
    }
    __shared__ float dsum[kGatherPairs][kGatherTex];
    int li = 0;   // this block's level (uniform)
    while (li + 1 < G.n && (int)blockIdx.x >= G.start[li + 1]) li++;
    const int level = G.lv[li];
    const DevLevel& L = m.lv[level];
    const int rate = rate0 && level == 0;
    float* const zq_copy = G.zq_copy[li];
    const int j = threadIdx.x % kGatherTex, q = threadIdx.x / kGatherTex;
    const int t = ((int)blockIdx.x - G.start[li]) * kGatherTex + j;
    const bool live = t < L.W * L.H;
    const int tt = live ? t : 0;
    const int tx = tt % L.W, ty = tt / L.W;
    const int* R = ranges + L.rng;
    const int x0 = R[tx], x1 = R[L.W + tx], y0 = R[2 * L.W + ty], y1 = R[2 * L.W + L.H + ty];
    const long long base = L.off + (long long)tt * L.C;
    const int blk = (ty / 8) * dct_bw + tx / 8;
    for (int k0 = 0; k0 < K; k0 += kGatherPairs) {
        const int k = k0 + q;
        if (live && k < K) {
            // the rectangle's values in raster order, loaded in groups and then added in order (the loads of
            // a group overlap; the sum stays one chain). A slot past the rectangle's end adds +0, which
            // leaves the sum as it is: the sum starts at +0 and a rounded sum is -0 only when both operands
            // are, so it is never -0. Rectangles up to 16 wide go in groups of kGatherRun values across row
            // ends, wider ones a row at a time in runs of 16; a one-pixel rectangle is one load.
            const float* dp = dpix + (size_t)k * m.npix;
            const int fw = x1 - x0, n = fw * (y1 - y0);
            float d = 0.0f;
            if (n == 1) {
                d += dp[(size_t)y0 * m.W + x0];
            } else if (fw <= 16) {
                int row = y0, col = 0;   // position of the group's first slot
                for (int s = 0; s < n; s += kGatherRun) {
                    float v[kGatherRun];
                    int r = row, cc = col;
#pragma unroll
                    for (int i = 0; i < kGatherRun; i++) {
                        v[i] = s + i < n ? dp[(size_t)r * m.W + x0 + cc] : 0.0f;
                        if (++cc == fw) { cc = 0; r++; }
                    }
                    row = r; col = cc;
#pragma unroll
                    for (int i = 0; i < kGatherRun; i++) d += v[i];
                }
            } else {
                // runs of 16 in raster order (a row's last run padded with +0), two buffers: the next run's loads are
                // in flight while the current run is added
                float va[16], vb[16];
                auto load_run = [&](float (&v)[16], int py, int px) {
                    const float* rw = dp + (size_t)py * m.W;
#pragma unroll
                    for (int i = 0; i < 16; i++) v[i] = px + i < x1 ? rw[px + i] : 0.0f;
                };
                auto step = [&](int& py, int& px) { px += 16; if (px >= x1) { px = x0; py++; } };
                int py = y0, px = x0;
                load_run(va, py, px);
                while (true) {
                    step(py, px);
                    if (py < y1) load_run(vb, py, px);
#pragma unroll
                    for (int i = 0; i < 16; i++) d += va[i];
                    if (py >= y1) break;
                    step(py, px);
                    if (py < y1) load_run(va, py, px);
#pragma unroll
                    for (int i = 0; i < 16; i++) d += vb[i];
                    if (py >= y1) break;
                }
            }
            dsum[q][j] = d;
        }
        __syncthreads();
        // the round's pairs in order on every channel of the texel (thread q takes channels q, q + 4, ...),
        // the channel's gradient in a register; after the last round the channel's Adam step
        if (live) {
            const int kn = min(K, k0 + kGatherPairs) - k0;
            const bool last = k0 + kGatherPairs >= K;
            for (int c = q; c < L.C; c += kGatherPairs) {
                const size_t i = (size_t)(base + c);
                float gc = (first && k0 == 0) ? 0.0f : grad[i];
                for (int kk = 0; kk < kn; kk++) {
                    const float ei = eps[(size_t)(k0 + kk) * m.nz + i];
                    gc = __builtin_fmaf(dsum[kk][j] * scale, ei, gc);
                    if (rate) {
                        const int32_t db = dbits[(size_t)(k0 + kk) * dct_n + (size_t)blk * L.C + c];
                        gc = __builtin_fmaf(__fmul_rn(__fmul_rn(rate_scale, (float)db), scale), ei, gc);
                    }
                }
                grad[i] = gc;
                if (adam && last) {
                    adam_at(z, zm, zv, i, gc, lr, c1, c2);
                    if (zq_copy) zq_copy[i] = z[i];   // a level the decode copy takes as it is
                }
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------- launchers
void launch_lat_eps(Impl& I, int k0, int K, unsigned mask) {
    ProfScope ps(I, "lat_eps");
    hipLaunchKernelGGL(k_lat_eps, dim3(blocks_for(I.nz, kTPB), K), dim3(kTPB), 0, I.stream, I.noise, I.dm, I.d.seed,
                       (uint32_t)I.lat_step_no, mask, k0, I.eps_lat, I.zgrad);
    NTC_CHECK(hipGetLastError());
}

void launch_lat_pair_valu(Impl& I, int K, float sigma, unsigned mask) {
    if (I.jit) {
        jit_launch(k_lat_pair<ShapeDefault>, I, "k_lat_pair", "", dim3(blocks_for(I.npix, kTPB), K), dim3(kTPB), 0, I.dm, I.w, I.zdec,
                   I.eps_lat, I.tgt, sigma, mask, I.dpix);
    } else dispatch_shape(I.dm, [&](auto s) {
        using S = decltype(s);
        hipLaunchKernelGGL(k_lat_pair<S>, dim3(blocks_for(I.npix, kTPB), K), dim3(kTPB), 0, I.stream, I.dm, I.w, I.zdec, I.eps_lat,
                           I.tgt, sigma, mask, I.dpix);
    });
    NTC_CHECK(hipGetLastError());
}

void launch_lat_gather(Impl& I, unsigned mask, int k0, int K, float scale, bool rate, float lr, int t, int ahead_K, float* zq_rest) {
    const float c1 = t > 0 ? 1.0f - powf(0.9f, (float)t) : 1.0f, c2 = t > 0 ? 1.0f - powf(0.999f, (float)t) : 1.0f;
    GatherLevels G{};
    size_t grid = 0;
    for (int l = 0; l < I.d.nlev; l++)
        if ((mask >> l) & 1u) {
            G.lv[G.n] = l;
            G.start[G.n] = (int)grid;
            G.zq_copy[G.n] = l > 0 ? zq_rest : nullptr;
            grid += (size_t)blocks_for((size_t)I.d.lv[l].W * I.d.lv[l].H, kGatherTex);
            G.n++;
        }
    G.start[G.n] = (int)grid;
    LatAhead ah{};
    ah.eb = 1;
    if (ahead_K > 0) {   // the next step's Gaussians: the range of entries the perturbed levels span
        ah.nt = I.noise; ah.seed = I.d.seed; ah.next_step = (uint32_t)(I.lat_step_no + 1); ah.mask = mask; ah.eps_next = I.eps_ahead;
        ah.lo = (long long)I.nz; ah.hi = 0;
        for (int l = 0; l < I.d.nlev; l++)
            if ((mask >> l) & 1u) {
                ah.lo = std::min<long long>(ah.lo, I.dm.lv[l].off);
                ah.hi = std::max<long long>(ah.hi, I.dm.lv[l].off + (long long)I.d.lv[l].W * I.d.lv[l].H * I.d.lv[l].C);
            }
        ah.eb = blocks_for((size_t)(ah.hi - ah.lo), kAheadPerBlock);
        grid += (size_t)ah.eb * (size_t)ahead_K;
    }
    if (grid > 0x7fffffff) {
        fprintf(stderr, "ntc_hip backend: latent gather launch of %zu blocks\n", grid);
        exit(1);
    }
    ProfScope ps(I, "lat_gather");
    hipLaunchKernelGGL(k_lat_gather, dim3((unsigned)grid), dim3(kGatherTex * kGatherPairs), 0, I.stream, I.dm, G, K,
                       scale, I.dpix, I.eps_lat,
                       I.ranges, rate ? 1 : 0, I.ddct.rate_scale, I.ddct.BW, I.ddct.n, rate ? I.dct_dbits + (size_t)k0 * I.ddct.n : nullptr,
                       I.zgrad, k0 == 0 ? 1 : 0, t > 0 ? 1 : 0, I.z, I.zm,
                       I.zv, lr, c1, c2, ah);
    NTC_CHECK(hipGetLastError());
}

void launch_qat_search(Impl& I) {
    const size_t ntx = (size_t)I.d.lv[0].W * I.d.lv[0].H;
    ProfScope ps(I, "qat_search");
    if (qat_on_matrix_cores(I)) {
        launch_qat_mfma(I);
        return;
    }
    if (I.jit) {
        jit_launch(k_qat_search<ShapeDefault>, I, "k_qat_search", "", dim3(blocks_for(ntx, kTPB)), dim3(kTPB), 0, I.dm, I.w, I.zdec,
                   I.tgt, I.ranges, I.qat_bits, I.qat_grid);
    } else dispatch_shape(I.dm, [&](auto s) {
        using S = decltype(s);
        hipLaunchKernelGGL(k_qat_search<S>, dim3(blocks_for(ntx, kTPB)), dim3(kTPB), 0, I.stream, I.dm, I.w, I.zdec, I.tgt, I.ranges,
                           I.qat_bits, I.qat_grid);
    });
    NTC_CHECK(hipGetLastError());
}

}   // namespace ntc_hip
