// Host-side state of one ntc_cuda::Trainer on gfx950 and the launchers of its kernels.
//
// Layout in HBM (all buffers owned by the trainer, allocated at init or grown on first use):
//   z, zq          latent shadow (Adam's) and the snapped decode copy (zq only with --qes / --dct-q);
//                  zdec aliases whichever every decode reads; (y, x, c) per level, levels concatenated
//   w              MLP parameters, per layer W[out][in] row-major then b[out]
//   wsets          2 x sets x P: the member weight vectors of one ES step (w +- sigma eps_i) or of one
//                  central-difference step (w with w_j +- h); read by the population evaluation
//   eps_mlp        N x P Gaussians of the last ES step (consumed by the weight update)
//   feat, btgt     the minibatch in structure-of-arrays form: feat[nin][Mcap], btgt[nout][Mcap]
//   eps_lat, dpix  K x nz latent Gaussians and K x W*H per-pixel loss differences of one latent step
//   tgt            W*H*nout target, interleaved as the caller's
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <stdlib.h>

#include <map>
#include <string>
#include <vector>

#include "device_common.hpp"
#include "ntc_cuda.h"
#include "ntc_hip.h"

#define NTC_CHECK(x)                                                                                          \
    do {                                                                                                      \
        hipError_t e_ = (x);                                                                                  \
        if (e_ != hipSuccess) {                                                                               \
            fprintf(stderr, "HIP error %s at %s:%d: %s\n", #x, __FILE__, __LINE__, hipGetErrorString(e_));   \
            exit(1);                                                                                          \
        }                                                                                                     \
    } while (0)

#include <atomic>

namespace ntc_hip {

// Every device allocation and release the library makes goes through these two, which count them
// (ntc_debug_device_allocations: a test that an entry point allocates nothing reads the count around it).
extern std::atomic<long long> g_device_allocs, g_device_frees;
template <class T>
hipError_t ntc_malloc(T** p, size_t bytes) {
    g_device_allocs.fetch_add(1, std::memory_order_relaxed);
    return hipMalloc((void**)p, bytes);
}
inline hipError_t ntc_free(void* p) {
    g_device_frees.fetch_add(1, std::memory_order_relaxed);
    return hipFree(p);
}

// --dct-q level 0 as the kernels see it (by value)
struct DevDct {
    int live, C, BW, BH, dc_step, deadzone, lo_w16, rate_es, rate_trunc, n;   // n = BW * BH * C
    float rate_scale;
    float lam_t16[16];
    float basis[64];     // [u * 8 + x], the caller's bit patterns
    int zigzag[64];
};

struct JitModuleSet;   // jit.cpp: the kernels specialised for one model shape

struct KernelTimes {
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
    double total_ms = 0.0;
    long long launches = 0;
};

}   // namespace ntc_hip

struct ntc_cuda::Trainer::Impl {
    ModelDesc d;
    ntc_hip::DevModel dm{};
    int device = 0;
    hipStream_t stream = nullptr;
    ntc_hip::NoiseFix noise{};
    int P = 0;
    size_t nz = 0, npix = 0;

    float *z = nullptr, *zq = nullptr, *zdec = nullptr, *zgrad = nullptr, *zm = nullptr, *zv = nullptr, *ztmp = nullptr;
    float *w = nullptr, *wgrad = nullptr, *wm = nullptr, *wv = nullptr;
    float *tgt = nullptr, *img = nullptr;
    float *feat = nullptr, *btgt = nullptr;
    int* bidx = nullptr;
    int Mcap = 0;
    // the minibatch's unperturbed first-layer pre-activations (H x Mcap + slack), for the population kernel that
    // shares them between a pair's members (k_pop_pair; pop_pair: the model's shape takes it)
    float* lay1 = nullptr;
    bool pop_pair = false;
    float* wsets = nullptr;
    size_t wsets_cap = 0;      // floats
    float* eps_mlp = nullptr;
    float* gpart = nullptr;    // segment partials of the ES update: ceil(max_pairs / 128) x P
    size_t gpart_cap = 0;
    double *part = nullptr, *dl = nullptr, *lsum = nullptr, *hh = nullptr;
    size_t part_cap = 0;
    int pairs_cap = 0;
    float *eps_lat = nullptr, *dpix = nullptr;   // one group of pairs of a latent step: Kcap x nz, Kcap x W*H
    int Kcap = 0;
    // The next latent step's Gaussians, drawn ahead by this step's last gather launch (extra blocks beside the
    // gather's) when the step ran as one group: valid for step ahead_step with ahead_K pairs (-1: none).
    float* eps_ahead = nullptr;
    int ahead_step = -1, ahead_K = 0;
    int lat_group = 0;         // pairs per latent group (0: as many as kLatGroupBytes of eps_lat + dpix hold)
    int Dcap = 0;              // pairs dct_dbits holds
    int* ranges = nullptr;     // per level: xb[W] xe[W] yb[H] ye[H] (pixel footprint of each texel row / column)
    float* qat_grid = nullptr; // 9 x 257
    int* qat_bits = nullptr;   // MAX_CH
    bool lv0_unit_cells = false;   // level 0 nearest at the image's size: every texel's cell is its own pixel
    bool valu_only = false;        // instrumentation: every stage on the VALU kernels (ntc_trainer_set_matrix_cores)

    bool qes = false;
    ntc_cuda::QesDesc* qes_dev = nullptr;
    ntc_cuda::QesDesc qes_h{};     // the host's copy of the last set_qes (which levels are live, at what depth)
    float* qgrid = nullptr;

    bool dct = false, dct_live = false, dct_rate_es = false, dct_rate_trunc = false;
    ntc_hip::DevDct ddct{};
    int16_t* dct_sym = nullptr;
    uint8_t* dct_code = nullptr;
    int* dct_step = nullptr;
    int32_t *dct_bits = nullptr, *dct_dbits = nullptr;   // dbits: K x n (pair k's bit differences), every pair of the step
    int* dct_tn = nullptr;     // per (block, channel) of the last snap: truncated ACs [n], then nonzero ACs before truncation [n]
    uint8_t* dct_probe_code = nullptr;   // the device probe's codes (n)
    float* dct_gain = nullptr;           // and block gains (n)
    int dct_evals = 0, dct_last_K = 0;
    int lat_last_K = 0;            // pairs of the last latent group (the rows of dpix it wrote: the step's last pairs)

    // print_stats (kernels_stats.hip): the quantized latent, the histograms and partial sums (grown on first use),
    // and the host's copy of the last histograms (ntc_trainer_debug_print_counts)
    float* zpost = nullptr; size_t zpost_cap = 0;
    double* st_part = nullptr; size_t st_part_cap = 0;
    unsigned *st_keys = nullptr, *st_hist = nullptr, *st_dct = nullptr;
    size_t st_keys_cap = 0, st_hist_cap = 0, st_dct_cap = 0;
    unsigned long long* st_sse = nullptr; size_t st_sse_cap = 0;
    std::vector<long long> st_counts, st_dct_counts;
    std::vector<float> st_lohi;

    int mlp_t = 0, lat_t = 0, lat_step_no = 0;
    int last_N = 0, last_M = 0, last_chunk = 1;
    bool last_fd = false;

    std::string dev_name, arch;
    int cus = 0, rt_ver = 0;
    std::string shape_name = "runtime";
    ntc_hip::JitModuleSet* jit = nullptr;   // kernels specialised at init for a shape shapes.hpp does not list

    bool profiling = false;
    std::string prof_only;     // comma-separated kernel families to time; empty = all
    int prof_every = 1;        // time one launch in this many of each family
    std::map<std::string, long long> prof_seen;   // launches of each family since profiling was switched on
    hipEvent_t ext_a = nullptr, ext_b = nullptr;   // a ProfScope's events for the one launch it wraps (launch_timed)
    std::map<std::string, ntc_hip::KernelTimes> times;
};

namespace ntc_hip {
using Impl = ntc_cuda::Trainer::Impl;

// profiling: events around the launches of a scope on the trainer's stream. A scope that wraps exactly one
// launch through launch_timed / jit_launch (`one`) hands its events to that launch, which records them with
// the kernel's own dispatch (the kernel's start and end, no marker packets on the stream: an event record
// between two kernels costs the stream several microseconds); any other scope records them around its work.
struct ProfScope {
    Impl& I; const char* name; hipEvent_t a = nullptr, b = nullptr;
    bool on, one;
    ProfScope(Impl& I_, const char* n, bool one_launch = false)
        : I(I_), name(n), on(I_.profiling && selected(I_.prof_only, n) && sampled(I_, n)), one(on && one_launch) {
        if (!on) return;
        NTC_CHECK(hipEventCreate(&a)); NTC_CHECK(hipEventCreate(&b));
        if (one) { I.ext_a = a; I.ext_b = b; }
        else NTC_CHECK(hipEventRecord(a, I.stream));
    }
    ~ProfScope() {
        if (!on) return;
        if (one) {
            if (I.ext_a) { fprintf(stderr, "ntc_hip backend: timed scope %s launched no kernel\n", name); exit(1); }
        } else {
            NTC_CHECK(hipEventRecord(b, I.stream));
        }
        I.times[name].pending.emplace_back(a, b);
    }
    static bool sampled(Impl& I, const char* n) { return I.prof_every <= 1 || I.prof_seen[n]++ % I.prof_every == 0; }
    static bool selected(const std::string& only, const char* n) {
        if (only.empty()) return true;
        const std::string key = "," + only + ",", item = "," + std::string(n) + ",";
        return key.find(item) != std::string::npos;
    }
};
void resolve_times(Impl& I);

inline int blocks_for(size_t n, int tpb) { return (int)((n + tpb - 1) / tpb); }

// a launch on the trainer's stream; inside a one-launch ProfScope the kernel's dispatch records the scope's events
template <class... P, class... A>
void launch_timed(void (*kern)(P...), Impl& I, dim3 grid, dim3 block, size_t shm, A&&... args) {
    if (I.ext_a) {
        hipExtLaunchKernelGGL(kern, grid, block, (uint32_t)shm, I.stream, I.ext_a, I.ext_b, 0u, std::forward<A>(args)...);
        I.ext_a = I.ext_b = nullptr;
    } else {
        hipLaunchKernelGGL(kern, grid, block, shm, I.stream, std::forward<A>(args)...);
    }
}

// noise tables (one pair per device, filled from the host C library on first use)
// the device's noise correction bits (built once per device); false with a reason if the host's
// C library cannot be reproduced
bool noise_fix_for_device(int device, NoiseFix& out, std::string& why);
std::vector<uint32_t> noise_fix_summary(const std::vector<uint32_t>& fix);

// kernels_mlp.hip
void launch_fill(Impl& I, float* p, size_t n, float v);
// the minibatch of step it; eps_pairs > 0: the same launch draws the step's Gaussians of that many pairs (EpsJob)
void launch_batch(Impl& I, int it, int M, int eps_pairs = 0, bool lay1 = false);
// whether this model's shape takes the pair-sharing population kernel (k_pop_pair; the trainer then keeps the
// minibatch's first layer, lay1), and whether an ES step with chunks of `chunk` slots does
bool pop_pair_possible(const Impl& I);
bool pop_pair_step(const Impl& I, int chunk);
// whether that kernel is the pixel-per-lane shapes' k_pop_pair_own
bool pop_pair_own_shape(const Impl& I);
void launch_perturb(Impl& I, int it, float sigma, int N);
// the Gaussians of one ES step (NS_MLP, it, pair, k) into eps_mlp, N x P
void launch_fd_sets(Impl& I, float h);
// which stages run on the matrix cores for this trainer's model
bool pop_on_matrix_cores(const Impl& I);
bool lat_pair_on_matrix_cores(const Impl& I);
bool qat_on_matrix_cores(const Impl& I);
void launch_qat_mfma(Impl& I);
// minibatch slots per population-evaluation block for a population of `pairs` pairs
int pop_chunk(const Impl& I, int pairs, int M);
void launch_pop_eval(Impl& I, int pairs, int M, int chunk, int chunks);
// the ES step's population evaluation on the matrix cores, staging the members' weights itself: with three or more
// chunks per pair it reads the step's Gaussians from eps_mlp, which the step's minibatch launch draws once
// (launch_batch with eps_pairs = N), else each chunk-0 block draws its pair's and writes them to eps_mlp
inline bool pop_reads_eps(int chunks) { return chunks >= 3; }
void launch_pop_eval_es(Impl& I, int it, float sigma, int N, int M, int chunk, int chunks);
void launch_pop_eval_valu(Impl& I, int pairs, int M, int chunk, int chunks);
void launch_es_update(Impl& I, int chunks, double norm, float sigma, int N, float lr, int t);
void launch_fd_finish(Impl& I, int chunks, double norm);
void launch_adam(Impl& I, float* theta, const float* g, float* m, float* v, size_t n, float lr, int t);
void launch_decode(Impl& I, const float* z);
void launch_debug_gauss(Impl& I, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index0, size_t n, float* out);
// the device's two noise factors for arguments k0 .. k0 + n - 1 (device buffers)
void launch_debug_factors(Impl& I, uint32_t k0, size_t n, float* rad, float* cosv);
void launch_copy_calibration(Impl& I, const float* src, float* dst, size_t n);

// kernels_latent.hip
// the Gaussians of pairs k0 .. k0 + K - 1 (rows 0 .. K - 1 of eps_lat); with k0 = 0 also clears the latent gradient
void launch_lat_eps(Impl& I, int k0, int K, unsigned mask);
void launch_lat_pair_valu(Impl& I, int K, float sigma, unsigned mask);
void launch_lat_pair(Impl& I, int K, float sigma, unsigned mask);
// the footprint gather of the levels in mask, in one launch, for the group of pairs k0 .. k0 + K - 1 (added to the
// gradient so far; rate: level 0's DCT rate term too); with t > 0 (the step's last group) also the Adam step t
// (learning rate lr) of their texels, and with zq_rest the new values of the levels past 0 in that decode copy;
// ahead_K > 0: extra blocks draw the next step's Gaussians of that many pairs
void launch_lat_gather(Impl& I, unsigned mask, int k0, int K, float scale, bool rate, float lr = 0.0f, int t = 0, int ahead_K = 0,
                       float* zq_rest = nullptr);
void launch_qat_search(Impl& I);

// kernels_quant.hip
void launch_qes_snap(Impl& I);
void launch_dct_clamp0(Impl& I);
// pull != 0: the level-0 shadow pulled toward the current plane first (a --dct-shadow-pull over the whole plane)
void launch_dct_snap(Impl& I, float pull = 0.0f);
void launch_dct_recon(Impl& I);
// the decoder sensitivity probe over the decode buffer: codes (and block gains, when gain != null) into device buffers
void launch_dct_probe(Impl& I, uint8_t* code, float* gain);
// per-block, per-texture 8-bit squared-error sums of the decode in img against the target (ceil(ew eh / 256) x 4)
void launch_u8_sse(Impl& I, int ew, int eh, unsigned long long* part);
// img rounded to 8 bits (save_png) into out (device, npix x nout)
void launch_pack_u8(Impl& I, uint8_t* out);
// decode the decode buffer and download it as 8-bit values
void decode_rgb8_impl(Impl& I, uint8_t* out);
// decode the decode buffer on the device and return mse_of's per-texture and weighted figures
void decode_error_impl(Impl& I, const float* z_host, int ew, int eh, double* tex_mse, double* weighted);
// noalloc.hip: decode_error with its partial sums in a static per-GPU scratch array (no allocation at call
// time); the array's device address is looked up once per GPU at init
bool noalloc_scratch_setup(int device, std::string& why);
void decode_error_noalloc_impl(Impl& I, const float* z_host, int ew, int eh, double* tex_mse, double* weighted);
// kernels_stats.hip: the progress line's figures from device histograms
void print_stats_impl(Impl& I, int qbits, int ew, int eh, ntc_print_stats* out);
void dct_probe_impl(Impl& I, uint8_t* code, float* gain);
void dct_refit_impl(Impl& I, uint8_t* code);
// the rate pass of pairs k0 .. k0 + K - 1 (Gaussians in rows 0 .. K - 1 of eps_lat; bit differences in rows k0 ..)
void launch_dct_rate_pairs(Impl& I, int k0, int K, float sigma);
void launch_shadow_pull(Impl& I, size_t off, size_t n, float f);

}   // namespace ntc_hip
