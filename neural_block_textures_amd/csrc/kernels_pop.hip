// Launchers of the matrix-core kernels of kern_pop.hpp.
#include "jit.hpp"
#include "kern_pop.hpp"
#include "shapes.hpp"
#include "trainer_impl.hpp"

namespace ntc_hip {

// every channel weight of the model is 1
static bool unit_cw(const Impl& I) {
    bool unit = true;
    for (int c = 0; c < I.dm.nout; c++) unit = unit && I.dm.cw[c] == 1.0f;
    return unit;
}

bool qat_on_matrix_cores(const Impl& I) {
    if (!I.lv0_unit_cells || I.valu_only) return false;
    if (I.jit) return jit_mfma(I);
    bool ok = false;
    dispatch_shape(I.dm, [&](auto s) { ok = MfmaShape<decltype(s)>::kOk; });
    return ok;
}

// the population and latent-pair evaluations on the matrix cores take 0 <= leak <= 1 (kActFold, kActMax)
bool pop_on_matrix_cores(const Impl& I) {
    if (I.valu_only || !(I.dm.leak >= 0.0f && I.dm.leak <= 1.0f)) return false;
    if (I.jit) return jit_mfma(I);
    bool ok = false;
    dispatch_shape(I.dm, [&](auto s) { ok = MfmaShape<decltype(s)>::kOk; });
    return ok;
}

#ifndef NTC_POP_MIN_BLOCKS
#define NTC_POP_MIN_BLOCKS 2048
#endif
int pop_chunk(const Impl& I, int pairs, int M) {
    if (pop_on_matrix_cores(I)) {
        // at least NTC_POP_MIN_BLOCKS blocks where the population allows, at least 256 slots per chunk
        const int want = std::max(1, std::min((NTC_POP_MIN_BLOCKS + pairs - 1) / pairs, M / 256));
        const int chunk = ((M + want - 1) / want + 15) & ~15;
        return std::max(chunk, 16);
    }
    return std::min(M, 1024);
}

template <class S, int Act, int From>
static void launch_pop_mfma(Impl& I, const PopSource& src, int pairs, int M, int chunk, int chunks) {
    auto kern = I.dm.clamp_out ? k_pop_mfma<S, Act, true, From> : k_pop_mfma<S, Act, false, From>;
    launch_timed(kern, I, dim3(pairs, chunks), dim3(64 * kPopWaves), 0, I.dm, src, M, I.Mcap, chunk, chunks, I.feat, I.btgt, I.part);
}

static void check_pop_launch(const Impl& I, int pairs, int chunk, int chunks) {
    if ((size_t)2 * pairs * chunks > I.part_cap) {
        fprintf(stderr, "ntc_hip backend: population evaluation needs %d partial sums, buffer holds %zu\n", 2 * pairs * chunks,
                I.part_cap);
        exit(1);
    }
    if (chunk % 16 != 0) {
        fprintf(stderr, "ntc_hip backend: matrix-core population evaluation needs 16-slot chunks (got %d)\n", chunk);
        exit(1);
    }
}

template <int From>
static void launch_pop_matrix(Impl& I, const PopSource& src, int pairs, int M, int chunk, int chunks) {
    if (I.jit) {   // the same choice of activation as below
        const int act = From == kSets ? kActMax : kActFold;
        jit_launch(k_pop_mfma<ShapeMaterial, kActFold, false, From>, I, "k_pop_mfma",
                   std::to_string(act) + (I.dm.clamp_out ? ", true, " : ", false, ") + std::to_string(From), dim3(pairs, chunks),
                   dim3(64 * kPopWaves), 0, I.dm, src, M, I.Mcap, chunk, chunks, I.feat, I.btgt, I.part);
        NTC_CHECK(hipGetLastError());
        return;
    }
    dispatch_shape(I.dm, [&](auto s) {
        using S = decltype(s);
        if constexpr (MfmaShape<S>::kOk) {
            // central differences compare members one weight apart (w_j +- h): their activations are the
            // reference's bit for bit; the ES members (w +- sigma eps) take the one-instruction folded form
            if constexpr (From == kSets) launch_pop_mfma<S, kActMax, From>(I, src, pairs, M, chunk, chunks);
            else launch_pop_mfma<S, kActFold, From>(I, src, pairs, M, chunk, chunks);
        }
    });
    NTC_CHECK(hipGetLastError());
}

void launch_pop_eval(Impl& I, int pairs, int M, int chunk, int chunks) {
    ProfScope ps(I, "pop_eval", pop_on_matrix_cores(I));   // the matrix path is one launch
    if (!pop_on_matrix_cores(I)) {
        if ((size_t)2 * pairs * chunks > I.part_cap) {
            fprintf(stderr, "ntc_hip backend: population evaluation needs %d partial sums, buffer holds %zu\n", 2 * pairs * chunks,
                    I.part_cap);
            exit(1);
        }
        launch_pop_eval_valu(I, pairs, M, chunk, chunks);
        return;
    }
    check_pop_launch(I, pairs, chunk, chunks);
    PopSource src{};
    src.wsets = I.wsets;
    launch_pop_matrix<kSets>(I, src, pairs, M, chunk, chunks);
}

// The pair-sharing population kernels (k_pop_pair, k_pop_pair_own) take the ES steps of the fixed shapes they support
// (pop_pair_possible: the trainer then keeps a first-layer array of H x Mcap floats) whose chunks' first layers stay
// in the L2 (pop_pair_step: H x chunk floats within 2 MiB of an XCD's 4 MiB; the blocks of one chunk run together,
// so an XCD's working set is about one chunk's minibatch). NTC_HIP_POP_PAIR=0 keeps k_pop_mfma for every step.
bool pop_pair_possible(const Impl& I) {
    if (I.jit || I.valu_only || !(I.dm.leak >= 0.0f && I.dm.leak <= 1.0f)) return false;
    const char* env = getenv("NTC_HIP_POP_PAIR");
    if (env && env[0] == '0') return false;
    bool ok = false;
    dispatch_shape(I.dm, [&](auto s) { ok = pop_pair_ok<decltype(s)>() || pop_pair_own_ok<decltype(s)>(); });
    return ok;
}

bool pop_pair_own_shape(const Impl& I) {
    bool own = false;
    dispatch_shape(I.dm, [&](auto s) { own = pop_pair_own_ok<decltype(s)>(); });
    return own;
}

bool pop_pair_step(const Impl& I, int chunk) {
    return I.pop_pair && pop_on_matrix_cores(I) && (size_t)I.d.hidden[0] * (size_t)chunk * sizeof(float) <= ((size_t)2 << 20);
}

template <int From>
static void launch_pop_pair(Impl& I, const PopSource& src, int N, int M, int chunk, int chunks) {
    const bool unit = unit_cw(I);
    dispatch_shape(I.dm, [&](auto s) {
        using S = decltype(s);
        if constexpr (pop_pair_ok<S>()) {
            auto kern = I.dm.clamp_out ? (unit ? k_pop_pair<S, true, From, true> : k_pop_pair<S, true, From, false>)
                                       : (unit ? k_pop_pair<S, false, From, true> : k_pop_pair<S, false, From, false>);
            launch_timed(kern, I, dim3(N, chunks), dim3(64 * kPopWaves), 0, I.dm, src, M, I.Mcap, chunk, chunks, I.feat, I.btgt,
                         (const float*)I.lay1, I.part);
        } else if constexpr (pop_pair_own_ok<S>()) {
            auto kern = I.dm.clamp_out ? (unit ? k_pop_pair_own<S, true, From, true> : k_pop_pair_own<S, true, From, false>)
                                       : (unit ? k_pop_pair_own<S, false, From, true> : k_pop_pair_own<S, false, From, false>);
            launch_timed(kern, I, dim3(N, chunks), dim3(64 * kPopWaves), 0, I.dm, src, M, I.Mcap, chunk, chunks, I.feat, I.btgt,
                         (const float*)I.lay1, I.part);
        }
    });
    NTC_CHECK(hipGetLastError());
}

void launch_pop_eval_es(Impl& I, int it, float sigma, int N, int M, int chunk, int chunks) {
    check_pop_launch(I, N, chunk, chunks);
    PopSource src{};
    src.nt = I.noise; src.seed = I.d.seed; src.step = (uint32_t)it; src.sigma = sigma;
    src.w0 = I.w; src.eps = I.eps_mlp;
    ProfScope ps(I, "pop_eval", true);
    if (pop_pair_step(I, chunk)) {   // the step's minibatch launch wrote the first layer
        if (pop_reads_eps(chunks)) launch_pop_pair<kReadEps>(I, src, N, M, chunk, chunks);
        else launch_pop_pair<kDraw>(I, src, N, M, chunk, chunks);
        return;
    }
    if (pop_reads_eps(chunks)) launch_pop_matrix<kReadEps>(I, src, N, M, chunk, chunks);   // drawn by the minibatch launch
    else launch_pop_matrix<kDraw>(I, src, N, M, chunk, chunks);
}

// rounds per wave of the latent pair kernel: lat_rounds_of(nin) (the shape's most; the compiled shape has
// nin inputs), one where two would leave the launch under 2048 blocks. A count above the compiled kernel's
// would leave pixels of every block unevaluated: refused.
static int lat_rounds_for(const Impl& I, int most, int K) {
    if (most < 1 || most > lat_rounds_of(I.dm.nin)) {
        fprintf(stderr, "ntc_hip backend: latent pair launch with %d rounds for a %d-input model (at most %d)\n", most, I.dm.nin,
                lat_rounds_of(I.dm.nin));
        exit(1);
    }
    if (most > 1 && (size_t)((I.npix + 511) / 512) * (size_t)K < 2048) return 1;
    return most;
}

bool lat_pair_on_matrix_cores(const Impl& I) { return pop_on_matrix_cores(I); }

template <class S, int Act, int Sh>
static auto lat_kernel(bool clamp, bool unit) {
    return clamp ? (unit ? k_lat_pair_mfma<S, Act, true, Sh, true> : k_lat_pair_mfma<S, Act, true, Sh, false>)
                 : (unit ? k_lat_pair_mfma<S, Act, false, Sh, true> : k_lat_pair_mfma<S, Act, false, Sh, false>);
}

template <class S, int Act>
static void launch_lat_mfma(Impl& I, int K, float sigma, unsigned mask) {
    // a step that perturbs level 1 only shares the first layer's level-0 and positional k-steps between the members
    constexpr int Sh = lat_shared_ksteps<S>();
    auto kern = lat_kernel<S, Act, 0>(I.dm.clamp_out, unit_cw(I));
    if constexpr (Sh > 0) {
        if (mask == 2u) kern = lat_kernel<S, Act, Sh>(I.dm.clamp_out, unit_cw(I));
    }
    static_assert(lat_rounds<S>() >= 1, "a latent pair kernel takes at least one round");
    const int rounds = lat_rounds_for(I, lat_rounds<S>(), K), pix = 256 * rounds;
    hipLaunchKernelGGL(kern, dim3((unsigned)((I.npix + pix - 1) / pix), K), dim3(256), 0, I.stream, I.dm, I.w, I.zdec,
                       I.eps_lat, I.tgt, sigma, mask, I.dpix, rounds);
}

void launch_lat_pair(Impl& I, int K, float sigma, unsigned mask) {
    ProfScope ps(I, "lat_pair");
    if (!lat_pair_on_matrix_cores(I)) {
        launch_lat_pair_valu(I, K, sigma, mask);
        return;
    }
    if (I.jit) {
        const int act = kActFold;
        const int rounds = lat_rounds_for(I, lat_rounds_of(I.dm.nin), K), pix = 256 * rounds;
        jit_launch(k_lat_pair_mfma<ShapeMaterial, kActFold, false>, I, "k_lat_pair_mfma",
                   std::to_string(act) + (I.dm.clamp_out ? ", true" : ", false"), dim3((unsigned)((I.npix + pix - 1) / pix), K), dim3(256), 0,
                   I.dm, I.w, I.zdec, I.eps_lat, I.tgt, sigma, mask, I.dpix, rounds);
        NTC_CHECK(hipGetLastError());
        return;
    }
    dispatch_shape(I.dm, [&](auto s) {
        using S = decltype(s);
        if constexpr (MfmaShape<S>::kOk) {
            launch_lat_mfma<S, kActFold>(I, K, sigma, mask);
        }
    });
    NTC_CHECK(hipGetLastError());
}

void launch_qat_mfma(Impl& I) {
    if (I.jit) {
        const float leak = I.dm.leak;
        const int act = leak >= 0.0f && leak <= 1.0f ? kActFold : kActAny;
        jit_launch(k_qat_mfma<ShapeMaterial, kActFold, false>, I, "k_qat_mfma", std::to_string(act) + (I.dm.clamp_out ? ", true" : ", false"),
                   dim3((unsigned)((I.npix + 255) / 256)),
                   dim3(256), 0, I.dm, I.w, I.zdec, I.tgt, I.qat_bits, I.qat_grid);
        NTC_CHECK(hipGetLastError());
        return;
    }
    dispatch_shape(I.dm, [&](auto s) {
        using S = decltype(s);
        if constexpr (MfmaShape<S>::kOk)
        {
            const float leak = I.dm.leak;
            const bool fold = leak >= 0.0f && leak <= 1.0f, unit = unit_cw(I);
            auto kern = I.dm.clamp_out ? (fold ? (unit ? k_qat_mfma<S, kActFold, true, true> : k_qat_mfma<S, kActFold, true, false>)
                                               : k_qat_mfma<S, kActAny, true>)
                                       : (fold ? (unit ? k_qat_mfma<S, kActFold, false, true> : k_qat_mfma<S, kActFold, false, false>)
                                               : k_qat_mfma<S, kActAny, false>);
            hipLaunchKernelGGL(kern, dim3((unsigned)((I.npix + 255) / 256)), dim3(256), 0, I.stream, I.dm, I.w, I.zdec, I.tgt,
                               I.qat_bits, I.qat_grid);
        }
    });
    NTC_CHECK(hipGetLastError());
}

}   // namespace ntc_hip
