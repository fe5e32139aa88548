// extern "C" entry points of libntc_hip.so: one per ntc_cuda::Trainer method (include/ntc_hip.h),
// plus the instrumentation helpers the tests and the benchmark use.
#include <stddef.h>
#include <string.h>

#include <string>
#include <vector>

#include "ntc_hip.h"
#include "jit.hpp"
#include "trainer_impl.hpp"

using ntc_cuda::Trainer;

// The C descriptors must be the C++ ones byte for byte.
#define NTC_SAME_FIELD(C, CPP, F) static_assert(offsetof(C, F) == offsetof(CPP, F), #C "." #F " is misplaced")
static_assert(sizeof(ntc_level_desc) == sizeof(ntc_cuda::LevelDesc), "LevelDesc layout");
NTC_SAME_FIELD(ntc_level_desc, ntc_cuda::LevelDesc, off);
NTC_SAME_FIELD(ntc_level_desc, ntc_cuda::LevelDesc, nearest);
static_assert(sizeof(ntc_model_desc) == sizeof(ntc_cuda::ModelDesc), "ModelDesc layout");
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, lv);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, npos);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, nin);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, hidden);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, leak);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, clamp_out);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, cw);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, wsum);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, qat_bits);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, qat_grid);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, qes_bits);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, dct_q);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, dct_basis);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, dct_zigzag);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, max_pairs);
NTC_SAME_FIELD(ntc_model_desc, ntc_cuda::ModelDesc, seed);
static_assert(sizeof(ntc_qes_desc) == sizeof(ntc_cuda::QesDesc), "QesDesc layout");
NTC_SAME_FIELD(ntc_qes_desc, ntc_cuda::QesDesc, lo);
NTC_SAME_FIELD(ntc_qes_desc, ntc_cuda::QesDesc, grid_off);
static_assert(sizeof(ntc_dct_desc) == sizeof(ntc_cuda::DctDesc), "DctDesc layout");
NTC_SAME_FIELD(ntc_dct_desc, ntc_cuda::DctDesc, rate_scale);
NTC_SAME_FIELD(ntc_dct_desc, ntc_cuda::DctDesc, lam_t16);
NTC_SAME_FIELD(ntc_dct_desc, ntc_cuda::DctDesc, deadzone);

struct ntc_trainer { Trainer t; };

static size_t copy_out(const std::string& s, char* buf, size_t cap) {
    if (buf && cap) { const size_t n = std::min(cap - 1, s.size()); memcpy(buf, s.data(), n); buf[n] = 0; }
    return s.size();
}

extern "C" {

ntc_trainer* ntc_trainer_create(void) { return new ntc_trainer; }
void ntc_trainer_destroy(ntc_trainer* t) { delete t; }

int ntc_trainer_init(ntc_trainer* t, const ntc_model_desc* d, const float* z, const float* p, const float* target, char* why,
                     size_t why_cap) {
    std::string reason;
    ntc_cuda::ModelDesc md;
    memcpy((void*)&md, d, sizeof(md));
    const bool ok = t->t.init(md, z, p, target, reason);
    copy_out(ok ? std::string() : reason, why, why_cap);
    return ok ? 1 : 0;
}
size_t ntc_trainer_banner(const ntc_trainer* t, char* buf, size_t cap) { return copy_out(t->t.banner(), buf, cap); }

void ntc_trainer_upload_model(ntc_trainer* t, const float* z, const float* p) { t->t.upload_model(z, p); }
void ntc_trainer_download_model(ntc_trainer* t, float* z, float* p) { t->t.download_model(z, p); }
void ntc_trainer_set_qes(ntc_trainer* t, const ntc_qes_desc* q, const float* grid, size_t grid_n) {
    t->t.set_qes(*reinterpret_cast<const ntc_cuda::QesDesc*>(q), grid, grid_n);
}
void ntc_trainer_snap_latent(ntc_trainer* t) { t->t.snap_latent(); }
void ntc_trainer_shadow_pull(ntc_trainer* t, size_t off, size_t n, float f) { t->t.shadow_pull(off, n, f); }
void ntc_trainer_download_zq(ntc_trainer* t, float* zq) { t->t.download_zq(zq); }
void ntc_trainer_set_dct(ntc_trainer* t, const ntc_dct_desc* d, const uint8_t* code, const int16_t* sym, const int* step) {
    t->t.set_dct(*reinterpret_cast<const ntc_cuda::DctDesc*>(d), code, sym, step);
}
void ntc_trainer_download_dct(ntc_trainer* t, int16_t* sym, uint8_t* code) { t->t.download_dct(sym, code); }
void ntc_trainer_download_dct_rate(ntc_trainer* t, int32_t* bits, int32_t* dbits_last_pair, int* ntrunc, int* nz_before, int* hits,
                                   int* evals) {
    t->t.download_dct_rate(bits, dbits_last_pair, ntrunc, nz_before, hits, evals);
}

void ntc_trainer_dct_probe(ntc_trainer* t, uint8_t* code, float* gain) { t->t.dct_probe(code, gain); }
void ntc_trainer_dct_refit(ntc_trainer* t, uint8_t* code) { t->t.dct_refit(code); }
void ntc_trainer_decode_rgb8(ntc_trainer* t, uint8_t* out) { t->t.decode_rgb8(out); }
void ntc_trainer_decode_error(ntc_trainer* t, const float* z_host, int ew, int eh, double* tex_mse, double* weighted) {
    t->t.decode_error(z_host, ew, eh, tex_mse, weighted);
}
void ntc_trainer_print_stats(ntc_trainer* t, int qbits, int ew, int eh, ntc_print_stats* out) {
    ntc_hip::print_stats_impl(*t->t.im, qbits, ew, eh, out);
}
size_t ntc_trainer_debug_print_counts(const ntc_trainer* t, long long* bitrate, size_t cap_b, float* lohi, long long* dct,
                                      size_t cap_d, size_t* n_dct) {
    const auto& I = *t->t.im;
    if (bitrate) memcpy(bitrate, I.st_counts.data(), std::min(cap_b, I.st_counts.size()) * sizeof(long long));
    if (lohi) memcpy(lohi, I.st_lohi.data(), std::min<size_t>(3 * 64 * 2, I.st_lohi.size()) * sizeof(float));
    if (dct) memcpy(dct, I.st_dct_counts.data(), std::min(cap_d, I.st_dct_counts.size()) * sizeof(long long));
    if (n_dct) *n_dct = I.st_dct_counts.size();
    return I.st_counts.size();
}
void ntc_trainer_decode_error_noalloc(ntc_trainer* t, const float* z_host, int ew, int eh, double* tex_mse, double* weighted) {
    ntc_hip::decode_error_noalloc_impl(*t->t.im, z_host, ew, eh, tex_mse, weighted);
}

void ntc_trainer_mlp_step(ntc_trainer* t, int it, float sigma, float lr, int N, int M) { t->t.mlp_step(it, sigma, lr, N, M); }
void ntc_trainer_mlp_step_fd(ntc_trainer* t, int it, float h, float lr, int M) { t->t.mlp_step_fd(it, h, lr, M); }
void ntc_trainer_reset_mlp_adam(ntc_trainer* t) { t->t.reset_mlp_adam(); }
void ntc_trainer_mlp_stats(ntc_trainer* t, double* batch_loss, double* diff_std) { t->t.mlp_stats(*batch_loss, *diff_std); }

void ntc_trainer_lat_step(ntc_trainer* t, int it, float sigma, float lr, int K) { t->t.lat_step(it, sigma, lr, K); }
void ntc_trainer_qat_search(ntc_trainer* t) { t->t.qat_search(); }
void ntc_trainer_decode_full(ntc_trainer* t, const float* z_host, float* img) { t->t.decode_full(z_host, img); }

size_t ntc_trainer_debug_last_batch(const ntc_trainer* t, int* bidx, size_t cap) {
    std::vector<int> v; t->t.debug_last_batch(v);
    if (bidx) memcpy(bidx, v.data(), std::min(cap, v.size()) * sizeof(int));
    return v.size();
}
size_t ntc_trainer_debug_last_dl(const ntc_trainer* t, double* dl, size_t cap) {
    std::vector<double> v; t->t.debug_last_dl(v);
    if (dl) memcpy(dl, v.data(), std::min(cap, v.size()) * sizeof(double));
    return v.size();
}
size_t ntc_trainer_debug_last_zgrad(const ntc_trainer* t, float* g, size_t cap) {
    std::vector<float> v; t->t.debug_last_zgrad(v);
    if (g) memcpy(g, v.data(), std::min(cap, v.size()) * sizeof(float));
    return v.size();
}

size_t ntc_trainer_debug_last_dpix(const ntc_trainer* t, float* d, size_t cap) {
    auto& I = *t->t.im;
    const size_t n = (size_t)I.lat_last_K * (size_t)I.npix;
    if (d && cap && n) {
        NTC_CHECK(hipMemcpyAsync(d, I.dpix, std::min(cap, n) * sizeof(float), hipMemcpyDeviceToHost, I.stream));
        NTC_CHECK(hipStreamSynchronize(I.stream));
    }
    return n;
}

size_t ntc_trainer_debug_last_losses(const ntc_trainer* t, double* lplus, double* lminus, size_t cap) {
    auto& I = *t->t.im;
    const size_t n = (size_t)I.last_N;
    if (!n) return 0;
    const size_t m = std::min(cap, n);
    const int chunks = (I.last_M + I.last_chunk - 1) / I.last_chunk;
    std::vector<double> part((size_t)2 * n * chunks);
    NTC_CHECK(hipMemcpyAsync(part.data(), I.part, part.size() * sizeof(double), hipMemcpyDeviceToHost, I.stream));
    NTC_CHECK(hipStreamSynchronize(I.stream));
    const double norm = 3.0 * (double)I.d.wsum * (double)I.last_M;
    for (size_t i = 0; i < m; i++) {
        double a = 0.0, b = 0.0;
        for (int c = 0; c < chunks; c++) { a += part[(2 * i) * chunks + c]; b += part[(2 * i + 1) * chunks + c]; }
        if (lplus) lplus[i] = a / norm;
        if (lminus) lminus[i] = b / norm;
    }
    return n;
}
size_t ntc_trainer_debug_last_wgrad(const ntc_trainer* t, float* g, size_t cap) {
    auto& I = *t->t.im;
    const size_t n = (size_t)I.P;
    if (g && cap) {
        NTC_CHECK(hipMemcpyAsync(g, I.wgrad, std::min(cap, n) * sizeof(float), hipMemcpyDeviceToHost, I.stream));
        NTC_CHECK(hipStreamSynchronize(I.stream));
    }
    return n;
}
size_t ntc_abi_sizeof(const char* name) {
    const std::string n = name ? name : "";
    if (n == "ntc_model_desc") return sizeof(ntc_model_desc);
    if (n == "ntc_qes_desc") return sizeof(ntc_qes_desc);
    if (n == "ntc_dct_desc") return sizeof(ntc_dct_desc);
    if (n == "ntc_level_desc") return sizeof(ntc_level_desc);
    if (n == "ntc_print_stats") return sizeof(ntc_print_stats);
    return 0;
}
long long ntc_trainer_nparams(const ntc_trainer* t) { return t->t.im->P; }
long long ntc_trainer_nz(const ntc_trainer* t) { return (long long)t->t.im->nz; }
void* ntc_trainer_stream(const ntc_trainer* t) { return (void*)t->t.im->stream; }
void ntc_trainer_synchronize(ntc_trainer* t) { if (t->t.im->stream) NTC_CHECK(hipStreamSynchronize(t->t.im->stream)); }

void ntc_trainer_set_profiling(ntc_trainer* t, int on) {
    auto& I = *t->t.im;
    ntc_hip::resolve_times(I);
    I.profiling = on != 0;
    if (on) { I.times.clear(); I.prof_seen.clear(); }
}
void ntc_trainer_set_profiling_every(ntc_trainer* t, int n) { t->t.im->prof_every = n > 1 ? n : 1; }
void ntc_trainer_set_profiling_only(ntc_trainer* t, const char* names) { t->t.im->prof_only = names ? names : ""; }
int ntc_trainer_on_matrix_cores(ntc_trainer* t, const char* stage) {
    const auto& I = *t->t.im;
    const std::string s = stage ? stage : "";
    if (s == "pop_eval") return ntc_hip::pop_on_matrix_cores(I) ? 1 : 0;
    if (s == "lat_pair") return ntc_hip::lat_pair_on_matrix_cores(I) ? 1 : 0;
    if (s == "qat_search") return ntc_hip::qat_on_matrix_cores(I) ? 1 : 0;
    if (s == "pop_pair" || s == "pop_pair_own") {
        const bool pair = ntc_hip::pop_pair_step(I, ntc_hip::pop_chunk(I, I.pairs_cap, I.Mcap));
        return (pair && (s == "pop_pair" || ntc_hip::pop_pair_own_shape(I))) ? 1 : 0;
    }
    return 0;
}

void ntc_trainer_set_matrix_cores(ntc_trainer* t, int on) { t->t.im->valu_only = on == 0; }
void ntc_trainer_set_lat_group(ntc_trainer* t, int pairs) { t->t.im->lat_group = pairs > 0 ? pairs : 0; }

int ntc_jit_compile_check(const ntc_model_desc* d, const char* arch, double* seconds, char* why, size_t why_cap) {
    ntc_hip::DevModel m{};
    m.nlev = d->nlev; m.npos = d->npos; m.nl = d->nhidden; m.nout = d->nout; m.nin = d->nin; m.leak = d->leak;
    m.fold_c = (1.0f - d->leak) / (1.0f + d->leak);
    m.clamp_out = d->clamp_out ? 1 : 0;
    for (int l = 0; l < d->nlev && l < ntc_hip::kMaxLevels; l++) m.lv[l].C = d->lv[l].C;
    for (int l = 0; l < d->nhidden && l < ntc_hip::kMaxHidden; l++) m.hidden[l] = d->hidden[l];
    std::string w;
    const bool ok = ntc_hip::jit_compile_only(m, arch ? arch : "gfx950", w, seconds);
    if (why && why_cap) snprintf(why, why_cap, "%s", w.c_str());
    return ok ? 1 : 0;
}

int ntc_trainer_kernel_time(ntc_trainer* t, const char* name, double* total_ms, long long* launches) {
    auto& I = *t->t.im;
    ntc_hip::resolve_times(I);
    auto it = I.times.find(name);
    if (it == I.times.end()) { *total_ms = 0.0; *launches = 0; return 0; }
    *total_ms = it->second.total_ms; *launches = it->second.launches;
    return 1;
}

void ntc_trainer_debug_gauss(ntc_trainer* t, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index0, size_t n, float* out) {
    auto& I = *t->t.im;
    float* d = nullptr;
    NTC_CHECK(ntc_hip::ntc_malloc(&d, std::max<size_t>(n, 1) * sizeof(float)));
    ntc_hip::launch_debug_gauss(I, stream, step, pair, index0, n, d);
    NTC_CHECK(hipMemcpyAsync(out, d, n * sizeof(float), hipMemcpyDeviceToHost, I.stream));
    NTC_CHECK(hipStreamSynchronize(I.stream));
    NTC_CHECK(ntc_hip::ntc_free(d));
}
void ntc_trainer_debug_copy_calibration(ntc_trainer* t, size_t n, int reps) {
    auto& I = *t->t.im;
    n &= ~(size_t)3;
    float *a = nullptr, *b = nullptr;
    NTC_CHECK(ntc_hip::ntc_malloc(&a, std::max<size_t>(n, 4) * sizeof(float)));
    NTC_CHECK(ntc_hip::ntc_malloc(&b, std::max<size_t>(n, 4) * sizeof(float)));
    NTC_CHECK(hipMemsetAsync(a, 0, n * sizeof(float), I.stream));
    for (int r = 0; r < reps; r++) ntc_hip::launch_copy_calibration(I, a, b, n);
    NTC_CHECK(hipStreamSynchronize(I.stream));
    NTC_CHECK(ntc_hip::ntc_free(a));
    NTC_CHECK(ntc_hip::ntc_free(b));
}
void ntc_trainer_debug_noise_factors(ntc_trainer* t, uint32_t k0, size_t n, float* rad, float* cosv) {
    auto& I = *t->t.im;
    const size_t total = (size_t)1 << 24;
    if ((size_t)k0 >= total) return;
    if (n > total - k0) n = total - k0;
    if (!n) return;
    float *dr = nullptr, *dc = nullptr;
    NTC_CHECK(ntc_hip::ntc_malloc(&dr, n * sizeof(float)));
    NTC_CHECK(ntc_hip::ntc_malloc(&dc, n * sizeof(float)));
    ntc_hip::launch_debug_factors(I, k0, n, dr, dc);
    if (rad) NTC_CHECK(hipMemcpyAsync(rad, dr, n * sizeof(float), hipMemcpyDeviceToHost, I.stream));
    if (cosv) NTC_CHECK(hipMemcpyAsync(cosv, dc, n * sizeof(float), hipMemcpyDeviceToHost, I.stream));
    NTC_CHECK(hipStreamSynchronize(I.stream));
    NTC_CHECK(ntc_hip::ntc_free(dr));
    NTC_CHECK(ntc_hip::ntc_free(dc));
}

void ntc_debug_device_allocations(long long* allocs, long long* frees) {
    if (allocs) *allocs = ntc_hip::g_device_allocs.load();
    if (frees) *frees = ntc_hip::g_device_frees.load();
}

}   // extern "C"
