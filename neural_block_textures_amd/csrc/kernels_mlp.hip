// MLP-side kernels of the gfx950 ES backend: minibatch draw, member weight sets, the population
// evaluation, the central-difference finish, the ES weight update with its Adam step, Adam and the decode.
//
// Reference semantics (main.cpp): MlpTrainer::draw_batch 1825-1833, MlpTrainer::step 1836-1876,
// MlpTrainer::step_fd 1890-1920, Adam::step 1799-1809, Decoder::decode_full 1712-1718.
#include "kern_valu.hpp"
#include "jit.hpp"
#include "shapes.hpp"
#include "trainer_impl.hpp"

namespace ntc_hip {


__global__ void __launch_bounds__(kTPB) k_fill(float* __restrict__ p, size_t n, float v) {
    const size_t i = (size_t)blockIdx.x * kTPB + threadIdx.x;
    if (i < n) p[i] = v;
}

// Member weights of one ES step: pair i, weight k -> w0 +- sigma * eps (one fused operation each,
// main.cpp:1856), and eps itself for the update. The noise is the counter draw (NS_MLP, it, i, k).
__global__ void __launch_bounds__(kTPB) k_perturb(NoiseFix nt, uint64_t seed, uint32_t step, int N, int P, float sigma,
                                                 const float* __restrict__ w0, float* __restrict__ wsets,
                                                 float* __restrict__ eps) {
    const long long t = (long long)blockIdx.x * kTPB + threadIdx.x;
    if (t >= (long long)N * P) return;
    const int i = (int)(t / P), k = (int)(t - (long long)i * P);
    const float e = gauss_at(nt, noise_head(seed, NS_MLP, step, (uint32_t)i), (uint64_t)k);
    eps[t] = e;
    const float w = w0[k];
    wsets[(size_t)(2 * i) * P + k] = __builtin_fmaf(sigma, e, w);
    wsets[(size_t)(2 * i + 1) * P + k] = __builtin_fmaf(-sigma, e, w);
}

// Weight sets of one central-difference step: set pair j < P has w_j + h and w_j - h (float-realized,
// main.cpp:1905), pair P holds two copies of w for the unperturbed loss; hh[j] = wp - wm in double.
__global__ void __launch_bounds__(kTPB) k_fd_sets(int P, float h, const float* __restrict__ w0, float* __restrict__ wsets,
                                                 double* __restrict__ hh) {
    const long long t = (long long)blockIdx.x * kTPB + threadIdx.x;
    if (t >= (long long)(P + 1) * P) return;
    const int j = (int)(t / P), k = (int)(t - (long long)j * P);
    const float w = w0[k];
    const bool hit = k == j;
    const float wp = w + h, wm = w - h;
    wsets[(size_t)(2 * j) * P + k] = hit ? wp : w;
    wsets[(size_t)(2 * j + 1) * P + k] = hit ? wm : w;
    if (hit) hh[j] = (double)wp - (double)wm;
}

// ES update direction (main.cpp:1868-1873): g[k] = sum over pairs of ((float)dl_i * scale) * eps_ik, one
// fused multiply-add per pair. The reference sums the N pairs of a weight in one sequential chain, which
// leaves only P threads for N * P reads; here block (weight tile, segment) runs four chains of kChain
// pairs, one per wave, and the chains are added in a fixed order (waves, then segments), so the sum is
// deterministic and differs from the single chain only in rounding.
// Each wave first finishes its chain's pair losses from the population partials (lane q: pair i0 + q,
// the member's chunk sums added in ascending order, divided by the loss norm; with a single chain the four
// waves share that work by quarters of the chunks): dl_i = l+ - l-, and the blocks of weight tile 0 store dl
// and the pair means for the statistics.
constexpr int kChain = 32;
// With one segment (N <= 128 pairs) the block's sum is the gradient: the block writes it and takes the
// weight's Adam step itself (k_es_grad_final's work, the same operations), and no second kernel runs.
__global__ void __launch_bounds__(kTPB) k_es_grad_part(int N, int P, float scale, const double* __restrict__ lpart, int chunks,
                                                      double norm, double* __restrict__ dl, double* __restrict__ lsum,
                                                      const float* __restrict__ eps, float* __restrict__ part,
                                                      float* __restrict__ grad, float* __restrict__ theta, float* __restrict__ m,
                                                      float* __restrict__ v, float lr, float c1, float c2) {
    __shared__ float lds[kTPB / 64][64];
    __shared__ double quarters[kTPB / 64][2][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int k = blockIdx.x * 64 + lane;
    const int i0 = (blockIdx.y * (kTPB / 64) + wave) * kChain, i1 = min(N, i0 + kChain);
    // the loads that do not wait for the pair losses go first: a full chain's Gaussians, and the Adam state of the
    // weight this lane updates
    const bool full = i1 - i0 == kChain && k < P;
    float e[kChain];
    if (full) {
#pragma unroll
        for (int q = 0; q < kChain; q++) e[q] = eps[(size_t)(i0 + q) * P + k];
    }
    const bool adam_here = gridDim.y == 1 && wave == 0 && k < P;
    float th = 0.0f, mk = 0.0f, vk = 0.0f;
    if (adam_here) { th = theta[k]; mk = m[k]; vk = v[k]; }
    float wl = 0.0f;   // lane q: ((float)dl_{i0 + q}) * scale
    if (N <= kChain) {
        // one chain, which wave 0 runs: the four waves add a quarter of each member's chunk sums (lane q: pair q),
        // all of a quarter's loads in flight before its adds, then wave 0 adds the quarters in order
        const int c4 = (chunks + 3) >> 2, j0 = min(chunks, wave * c4), j1 = min(chunks, j0 + c4);
        double lp = 0.0, lm = 0.0;
        if (lane < N) {
            const double* pp = lpart + (size_t)(2 * lane) * chunks;
            const double* pm = pp + chunks;
            int j = j0;
            for (; j + 16 <= j1; j += 16) {
                double a[16], b[16];
#pragma unroll
                for (int q = 0; q < 16; q++) { a[q] = pp[j + q]; b[q] = pm[j + q]; }
#pragma unroll
                for (int q = 0; q < 16; q++) { lp += a[q]; lm += b[q]; }
            }
            for (; j < j1; j++) { lp += pp[j]; lm += pm[j]; }
        }
        quarters[wave][0][lane] = lp;
        quarters[wave][1][lane] = lm;
        __syncthreads();
        if (wave == 0 && lane < N) {
            lp = ((quarters[0][0][lane] + quarters[1][0][lane]) + quarters[2][0][lane]) + quarters[3][0][lane];
            lm = ((quarters[0][1][lane] + quarters[1][1][lane]) + quarters[2][1][lane]) + quarters[3][1][lane];
            lp /= norm; lm /= norm;
            const double d = lp - lm;
            if (blockIdx.x == 0) { dl[lane] = d; lsum[lane] = 0.5 * (lp + lm); }
            wl = __fmul_rn((float)d, scale);
        }
    } else if (i0 + lane < i1) {
        const int i = i0 + lane;
        // the member's chunk sums in ascending order, loaded 8 at a time (one chain of adds each)
        const double* pp = lpart + (size_t)(2 * i) * chunks;
        const double* pm = pp + chunks;
        double lp = 0.0, lm = 0.0;
        int j = 0;
        for (; j + 8 <= chunks; j += 8) {
            double a[8], b[8];
#pragma unroll
            for (int q = 0; q < 8; q++) { a[q] = pp[j + q]; b[q] = pm[j + q]; }
#pragma unroll
            for (int q = 0; q < 8; q++) { lp += a[q]; lm += b[q]; }
        }
        for (; j < chunks; j++) { lp += pp[j]; lm += pm[j]; }
        lp /= norm; lm /= norm;
        const double d = lp - lm;
        if (blockIdx.x == 0) { dl[i] = d; lsum[i] = 0.5 * (lp + lm); }
        wl = __fmul_rn((float)d, scale);
    }
    float g = 0.0f;
    if (k < P) {
        if (full) {   // a full chain: its loads were issued ahead of the dependent fma chain
#pragma unroll
            for (int q = 0; q < kChain; q++) g = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), q)), e[q], g);
        } else {
            for (int i = i0; i < i1; i++)
                g = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), i - i0)), eps[(size_t)i * P + k], g);
        }
    }
    lds[wave][lane] = g;
    __syncthreads();
    if (wave == 0 && k < P) {
        float s = lds[0][lane];
#pragma unroll
        for (int q = 1; q < kTPB / 64; q++) s += lds[q][lane];
        if (adam_here) {
            grad[k] = s;
            adam_vals(th, mk, vk, s, lr, c1, c2);
            theta[k] = th; m[k] = mk; v[k] = vk;
        } else {
            part[(size_t)blockIdx.y * P + k] = s;
        }
    }
}
// the segments added in order, then Adam on the weight
__global__ void __launch_bounds__(kTPB) k_es_grad_final(int P, int segs, const float* __restrict__ part, float* __restrict__ grad,
                                                       float* __restrict__ theta, float* __restrict__ m, float* __restrict__ v, float lr,
                                                       float c1, float c2) {
    const int k = blockIdx.x * kTPB + threadIdx.x;
    if (k >= P) return;
    float g = part[k];
#pragma unroll 8
    for (int s = 1; s < segs; s++) g += part[(size_t)s * P + k];
    grad[k] = g;
    adam_at(theta, m, v, (size_t)k, g, lr, c1, c2);
}

// Central differences: dl_j = L(w_j + h) - L(w_j - h), g_j = dl_j / hh_j; pair P gives L(w).
__global__ void __launch_bounds__(kTPB) k_fd_finish(const double* __restrict__ part, int chunks, int P, double norm,
                                                   const double* __restrict__ hh, double* __restrict__ dl,
                                                   double* __restrict__ lsum, float* __restrict__ grad) {
    const int j = blockIdx.x * kTPB + threadIdx.x;
    if (j > P) return;
    double lp = 0.0, lm = 0.0;
    for (int c = 0; c < chunks; c++) { lp += part[(size_t)(2 * j) * chunks + c]; lm += part[(size_t)(2 * j + 1) * chunks + c]; }
    lp /= norm; lm /= norm;
    if (j == P) { lsum[0] = lp; return; }
    const double d = lp - lm;
    dl[j] = d;
    grad[j] = (float)(d / hh[j]);
}

// Adam (main.cpp:1799-1809): m = fma(b1, m, (1 - b1) g), v = fma(b2, v, ((1 - b2) g) g),
// theta -= (lr m^) / (sqrt(v^) + eps); c1, c2 come from the host's powf.
__global__ void __launch_bounds__(kTPB) k_adam(float* __restrict__ theta, const float* __restrict__ g, float* __restrict__ m,
                                              float* __restrict__ v, size_t n, float lr, float c1, float c2) {
    const size_t i = (size_t)blockIdx.x * kTPB + threadIdx.x;
    if (i >= n) return;
    adam_at(theta, m, v, i, g[i], lr, c1, c2);
}

// A plain copy of known size, the reference point that turns the memory counters of a profile
// into bytes (n4 float4 values read once and written once).
__global__ void __launch_bounds__(kTPB) k_copy_calibration(const float4* __restrict__ src, float4* __restrict__ dst, size_t n4) {
    for (size_t i = (size_t)blockIdx.x * kTPB + threadIdx.x; i < n4; i += (size_t)gridDim.x * kTPB) dst[i] = src[i];
}

void launch_copy_calibration(Impl& I, const float* src, float* dst, size_t n) {
    const size_t n4 = n / 4;
    ProfScope ps(I, "copy_calibration");
    hipLaunchKernelGGL(k_copy_calibration, dim3((unsigned)std::min<size_t>(blocks_for(n4, kTPB), 8192)), dim3(kTPB), 0, I.stream,
                       (const float4*)src, (float4*)dst, n4);
    NTC_CHECK(hipGetLastError());
}

// A decode rounded to 8 bits as save_png writes it (lround of the [0, 1]-clamped value times 255).
__global__ void __launch_bounds__(kTPB) k_pack_u8(const float* __restrict__ img, size_t n, uint8_t* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * kTPB + threadIdx.x;
    if (i < n) out[i] = (uint8_t)(int)roundf(__fmul_rn(fminf(1.0f, fmaxf(0.0f, img[i])), 255.0f));
}

// The printed error of a decode (mse_of, main.cpp:1764-1788): both images rounded to 8 bits as save_png
// does (lround of the [0, 1]-clamped value times 255), the squared integer differences summed per
// texture over the evaluation extent ew x eh. Integer sums: exact and independent of order; one
// 64-bit partial per block and texture.
__global__ void __launch_bounds__(kTPB) k_u8_sse(const float* __restrict__ img, const float* __restrict__ tgt, int W, int ew, int eh,
                                                int nout, unsigned long long* __restrict__ part) {
    __shared__ unsigned long long red[kTPB / 64][4];
    const int T = nout / 3;
    const int i = blockIdx.x * kTPB + threadIdx.x;
    unsigned long long s[4] = { 0, 0, 0, 0 };
    if (i < ew * eh) {
        const size_t p = (size_t)(i / ew) * W + (i % ew);
        for (int t = 0; t < T; t++)
            for (int c = 0; c < 3; c++) {
                const float x = img[p * nout + 3 * t + c], y = tgt[p * nout + 3 * t + c];
                const int xi = (int)roundf(__fmul_rn(fminf(1.0f, fmaxf(0.0f, x)), 255.0f));
                const int yi = (int)roundf(__fmul_rn(fminf(1.0f, fmaxf(0.0f, y)), 255.0f));
                s[t] += (unsigned long long)((xi - yi) * (xi - yi));
            }
    }
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        unsigned long long v = s[t];
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        if (lane == 0) red[wid][t] = v;
    }
    __syncthreads();
    if (threadIdx.x < 4) {
        unsigned long long v = 0;
        for (int q = 0; q < kTPB / 64; q++) v += red[q][threadIdx.x];
        part[(size_t)blockIdx.x * 4 + threadIdx.x] = v;
    }
}

__global__ void __launch_bounds__(kTPB) k_debug_factors(NoiseFix nt, uint32_t k0, size_t n, float* __restrict__ rad,
                                                       float* __restrict__ cosv) {
    const size_t i = (size_t)blockIdx.x * kTPB + threadIdx.x;
    if (i >= n) return;
    rad[i] = nm_radius(nt, k0 + (uint32_t)i);
    cosv[i] = nm_cosine(nt, k0 + (uint32_t)i);
}

__global__ void __launch_bounds__(kTPB) k_debug_gauss(NoiseFix nt, uint64_t head, uint64_t index0, size_t n, float* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * kTPB + threadIdx.x;
    if (i < n) out[i] = gauss_at(nt, head, index0 + i);
}

// ---------------------------------------------------------------- launchers
void launch_fill(Impl& I, float* p, size_t n, float v) {
    if (!n) return;
    hipLaunchKernelGGL(k_fill, dim3(blocks_for(n, kTPB)), dim3(kTPB), 0, I.stream, p, n, v);
    NTC_CHECK(hipGetLastError());
}

void launch_batch(Impl& I, int it, int M, int eps_pairs, bool lay1) {
    const uint64_t head = noise_head(I.d.seed, NS_BATCH_PIX, (uint32_t)it, 0);
    const unsigned nb = blocks_for(M, kTPB);
    EpsJob ej{ I.noise, I.d.seed, (uint32_t)it, eps_pairs, I.P, I.eps_mlp, (int)nb };
    if (lay1 && !I.lay1) {
        fprintf(stderr, "ntc_hip backend: minibatch launch asked for the first layer without its buffer\n");
        exit(1);
    }
    Lay1Job l1{ lay1 ? I.w : nullptr, lay1 ? I.lay1 : nullptr };
    const unsigned grid = nb + (eps_pairs > 0 ? blocks_for((size_t)eps_pairs * I.P, kTPB) : 0u);
    ProfScope ps(I, "batch");
    if (I.jit) {
        jit_launch(k_batch<ShapeDefault>, I, "k_batch", "", dim3(grid), dim3(kTPB), 0, I.dm, head, M, I.Mcap, I.zdec,
                   I.tgt, I.bidx, I.feat, I.btgt, ej, l1);
    } else dispatch_shape(I.dm, [&](auto s) {
        using S = decltype(s);
        hipLaunchKernelGGL(k_batch<S>, dim3(grid), dim3(kTPB), 0, I.stream, I.dm, head, M, I.Mcap, I.zdec, I.tgt,
                           I.bidx, I.feat, I.btgt, ej, l1);
    });
    NTC_CHECK(hipGetLastError());
}

void launch_perturb(Impl& I, int it, float sigma, int N) {
    const size_t n = (size_t)N * I.P;
    ProfScope ps(I, "perturb");
    hipLaunchKernelGGL(k_perturb, dim3(blocks_for(n, kTPB)), dim3(kTPB), 0, I.stream, I.noise, I.d.seed, (uint32_t)it, N, I.P,
                       sigma, I.w, I.wsets, I.eps_mlp);
    NTC_CHECK(hipGetLastError());
}

void launch_fd_sets(Impl& I, float h) {
    const size_t n = (size_t)(I.P + 1) * I.P;
    ProfScope ps(I, "fd_sets");
    hipLaunchKernelGGL(k_fd_sets, dim3(blocks_for(n, kTPB)), dim3(kTPB), 0, I.stream, I.P, h, I.w, I.wsets, I.hh);
    NTC_CHECK(hipGetLastError());
}

void launch_pop_eval_valu(Impl& I, int pairs, int M, int chunk, int chunks) {
    if (I.jit) {
        jit_launch(k_pop_eval<ShapeDefault>, I, "k_pop_eval", "", dim3(pairs, chunks), dim3(kTPB), 0, I.dm, I.wsets, M, I.Mcap, chunk,
                   chunks, I.feat, I.btgt, I.part);
    } else dispatch_shape(I.dm, [&](auto s) {
        using S = decltype(s);
        hipLaunchKernelGGL(k_pop_eval<S>, dim3(pairs, chunks), dim3(kTPB), 0, I.stream, I.dm, I.wsets, M, I.Mcap, chunk, chunks,
                           I.feat, I.btgt, I.part);
    });
    NTC_CHECK(hipGetLastError());
}

// The pair losses, the update direction and the Adam step of an ES step (main.cpp:1862-1874)
void launch_es_update(Impl& I, int chunks, double norm, float sigma, int N, float lr, int t) {
    const float scale = 1.0f / (2.0f * (float)N * sigma);
    const float c1 = 1.0f - powf(0.9f, (float)t), c2 = 1.0f - powf(0.999f, (float)t);
    const int per_block = kChain * (kTPB / 64);
    const int segs = (N + per_block - 1) / per_block;
    if ((size_t)segs * I.P > I.gpart_cap) {   // sized at init for max_pairs; N never exceeds it
        fprintf(stderr, "ntc_hip backend: ES update partials exceed their buffer\n");
        exit(1);
    }
    ProfScope ps(I, "es_grad");
    float* part = I.gpart;
    hipLaunchKernelGGL(k_es_grad_part, dim3(blocks_for(I.P, 64), segs), dim3(kTPB), 0, I.stream, N, I.P, scale, I.part, chunks, norm,
                       I.dl, I.lsum, I.eps_mlp, part, I.wgrad, I.w, I.wm, I.wv, lr, c1, c2);
    NTC_CHECK(hipGetLastError());
    if (segs > 1) {
        hipLaunchKernelGGL(k_es_grad_final, dim3(blocks_for(I.P, kTPB)), dim3(kTPB), 0, I.stream, I.P, segs, part, I.wgrad, I.w, I.wm,
                           I.wv, lr, c1, c2);
        NTC_CHECK(hipGetLastError());
    }
}

void launch_fd_finish(Impl& I, int chunks, double norm) {
    hipLaunchKernelGGL(k_fd_finish, dim3(blocks_for(I.P + 1, kTPB)), dim3(kTPB), 0, I.stream, I.part, chunks, I.P, norm, I.hh,
                       I.dl, I.lsum, I.wgrad);
    NTC_CHECK(hipGetLastError());
}

void launch_adam(Impl& I, float* theta, const float* g, float* m, float* v, size_t n, float lr, int t) {
    const float c1 = 1.0f - powf(0.9f, (float)t), c2 = 1.0f - powf(0.999f, (float)t);
    ProfScope ps(I, "adam");
    hipLaunchKernelGGL(k_adam, dim3(blocks_for(n, kTPB)), dim3(kTPB), 0, I.stream, theta, g, m, v, n, lr, c1, c2);
    NTC_CHECK(hipGetLastError());
}

void launch_decode(Impl& I, const float* z) {
    ProfScope ps(I, "decode");
    if (I.jit) {
        jit_launch(k_decode<ShapeDefault>, I, "k_decode", "", dim3(blocks_for(I.npix, kTPB)), dim3(kTPB), 0, I.dm, I.w, z, I.img);
    } else dispatch_shape(I.dm, [&](auto s) {
        using S = decltype(s);
        hipLaunchKernelGGL(k_decode<S>, dim3(blocks_for(I.npix, kTPB)), dim3(kTPB), 0, I.stream, I.dm, I.w, z, I.img);
    });
    NTC_CHECK(hipGetLastError());
}

void launch_debug_gauss(Impl& I, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index0, size_t n, float* out) {
    if (!n) return;
    const uint64_t head = noise_head(I.d.seed, stream, step, pair);
    hipLaunchKernelGGL(k_debug_gauss, dim3(blocks_for(n, kTPB)), dim3(kTPB), 0, I.stream, I.noise, head, index0, n, out);
    NTC_CHECK(hipGetLastError());
}

void launch_debug_factors(Impl& I, uint32_t k0, size_t n, float* rad, float* cosv) {
    hipLaunchKernelGGL(k_debug_factors, dim3(blocks_for(n, kTPB)), dim3(kTPB), 0, I.stream, I.noise, k0, n, rad, cosv);
    NTC_CHECK(hipGetLastError());
}

void launch_u8_sse(Impl& I, int ew, int eh, unsigned long long* part) {
    hipLaunchKernelGGL(k_u8_sse, dim3(blocks_for((size_t)ew * eh, kTPB)), dim3(kTPB), 0, I.stream, I.img, I.tgt, I.d.W, ew, eh, I.d.nout,
                       part);
    NTC_CHECK(hipGetLastError());
}

void launch_pack_u8(Impl& I, uint8_t* out) {
    ProfScope ps(I, "pack_u8");
    const size_t n = (size_t)I.npix * I.d.nout;
    hipLaunchKernelGGL(k_pack_u8, dim3(blocks_for(n, kTPB)), dim3(kTPB), 0, I.stream, I.img, n, out);
    NTC_CHECK(hipGetLastError());
}

}   // namespace ntc_hip
