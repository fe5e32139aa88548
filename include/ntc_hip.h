/* C ABI of the MI355X (gfx950) ES training backend, exported by libntc_hip.so.
 *
 * One entry point per method of ntc_cuda::Trainer (include/ntc_cuda.h, which is
 * declaration-compatible with the reference's cuda/ntc_cuda.h); each comment names the reference
 * declaration it replaces. Plain C: opaque handle, plain pointers and sizes, host buffers only.
 * The descriptor structs have exactly the layout of their C++ counterparts in ntc_cuda.h
 * (checked with static_assert in the library), so a caller may pass either.
 *
 * Error behaviour follows the reference: ntc_trainer_init returns 0 and writes a reason for a
 * model outside the envelope; any other misuse or device error prints a message and exits.
 */
#pragma once
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NTC_MAX_LEVELS 3
#define NTC_MAX_POS 16
#define NTC_MAX_OUT 12
#define NTC_MAX_HIDDEN 8
#define NTC_MAX_CH 16
#define NTC_MAX_QES_CH 64
#define NTC_MAX_DCT_CH 4

typedef struct ntc_level_desc { int W, H, C; size_t off; bool nearest; } ntc_level_desc;   /* LevelDesc, cuda/ntc_cuda.h:25 */
typedef struct ntc_pos_desc { int kind; } ntc_pos_desc;                                      /* PosDesc, cuda/ntc_cuda.h:26 */

typedef struct ntc_model_desc {                     /* ModelDesc, cuda/ntc_cuda.h:29-52 */
    int W, H;
    int T;
    int nlev; ntc_level_desc lv[NTC_MAX_LEVELS];
    int npos; ntc_pos_desc pos[NTC_MAX_POS];
    int nin, nout;
    int nhidden; int hidden[NTC_MAX_HIDDEN];
    float leak;
    bool clamp_out;
    float cw[NTC_MAX_OUT];
    float wsum;
    int qat_bits[NTC_MAX_CH];
    int qat;
    const float* qat_grid;
    int qes_bits[NTC_MAX_LEVELS];
    int dct, dct_C, dct_N, dct_dc_step;
    int dct_q[NTC_MAX_DCT_CH];
    const float* dct_basis;
    const int* dct_zigzag;
    int max_pairs;
    int max_batch;
    uint64_t seed;
} ntc_model_desc;

typedef struct ntc_qes_desc {                       /* QesDesc, cuda/ntc_cuda.h:57-63 */
    int bits[NTC_MAX_LEVELS];
    int live;
    int frozen;
    float lo[NTC_MAX_LEVELS][NTC_MAX_QES_CH], hi[NTC_MAX_LEVELS][NTC_MAX_QES_CH], range[NTC_MAX_LEVELS][NTC_MAX_QES_CH];
    int grid_off[NTC_MAX_LEVELS][NTC_MAX_QES_CH];
} ntc_qes_desc;

typedef struct ntc_dct_desc {                       /* DctDesc, cuda/ntc_cuda.h:68-76 */
    int live, C, BW, BH, N, dc_step;
    int rate_es, rate_trunc; float rate_scale; float lam_t16[16];
    int lo_w16;
    int deadzone;
} ntc_dct_desc;

typedef struct ntc_trainer ntc_trainer;             /* an ntc_cuda::Trainer */

/* Trainer::Trainer / ~Trainer (cuda/ntc_cuda.h:80-81) */
ntc_trainer* ntc_trainer_create(void);
void ntc_trainer_destroy(ntc_trainer* t);
/* Trainer::init (cuda/ntc_cuda.h:85): 1 on success; 0 with a reason in why[0..why_cap) */
int ntc_trainer_init(ntc_trainer* t, const ntc_model_desc* d, const float* z, const float* p, const float* target,
                     char* why, size_t why_cap);
/* Trainer::banner (cuda/ntc_cuda.h:86): writes at most cap bytes (NUL-terminated), returns the full length */
size_t ntc_trainer_banner(const ntc_trainer* t, char* buf, size_t cap);

/* Trainer::upload_model / download_model (cuda/ntc_cuda.h:88-89): z = nz floats, p = P floats */
void ntc_trainer_upload_model(ntc_trainer* t, const float* z, const float* p);
void ntc_trainer_download_model(ntc_trainer* t, float* z, float* p);
/* Trainer::set_qes / snap_latent / shadow_pull / download_zq (cuda/ntc_cuda.h:93-96). snap_latent and shadow_pull
 * touch device memory only and return once their kernels are enqueued on the trainer's stream, as the
 * reference's do (cuda/ntc_cuda.cu:978-988); every call that copies to or from the host waits for them. */
void ntc_trainer_set_qes(ntc_trainer* t, const ntc_qes_desc* q, const float* grid, size_t grid_n);
void ntc_trainer_snap_latent(ntc_trainer* t);
void ntc_trainer_shadow_pull(ntc_trainer* t, size_t off, size_t n, float f);
void ntc_trainer_download_zq(ntc_trainer* t, float* zq);
/* Trainer::set_dct / download_dct / download_dct_rate (cuda/ntc_cuda.h:100-106) */
void ntc_trainer_set_dct(ntc_trainer* t, const ntc_dct_desc* d, const uint8_t* code, const int16_t* sym, const int* step);
void ntc_trainer_download_dct(ntc_trainer* t, int16_t* sym, uint8_t* code);
void ntc_trainer_download_dct_rate(ntc_trainer* t, int32_t* bits, int32_t* dbits_last_pair, int* ntrunc, int* nz_before,
                                   int* hits, int* evals);
/* The decoder sensitivity probe of a --dct-q level 0 on the device. No counterpart in the reference's
 * backend: it replaces the host's dct_probe_codes (main.cpp:1001-1032), which needs the model downloaded
 * first. Codes (BW*BH*C, [block][channel]) and, if gain is not null, the block gains of the current decode
 * buffer and weights. Requires --dct-q in the model description. */
void ntc_trainer_dct_probe(ntc_trainer* t, uint8_t* code, float* gain);
/* Decoder::dct_refit (main.cpp:1672-1680) on the device: probe, replace the codes, re-snap level 0 from the
 * shadow; the new codes are returned if code is not null (download_dct gives the symbols). Replaces the
 * reference's download + host refit + set_dct (main.cpp:4110-4120). Requires a prior set_dct. */
void ntc_trainer_dct_refit(ntc_trainer* t, uint8_t* code);
/* The printed error of the current model (mse_of, main.cpp:1764-1788) without a download: the decode
 * buffer - or z_host (nz floats, as decode_full; the post-hoc quantized latent of the print path's
 * second figure, main.cpp:4172-4174) - decoded on the device, both images rounded to 8 bits as save_png
 * does, squared differences summed exactly per texture over the extent ew x eh (0 = the whole image).
 * tex_mse[T] = SSE_t / (3 ew eh), *weighted = sum_t w_t SSE_t / (3 wsum ew eh), with w_t = cw[3 t].
 * No counterpart in the reference's backend (its print path downloads the model and decodes on the
 * host, main.cpp:4155-4174). */
void ntc_trainer_decode_error(ntc_trainer* t, const float* z_host, int ew, int eh, double* tex_mse, double* weighted);
/* ntc_trainer_decode_error with no allocation at call time (no hipMalloc / hipFree, no allocating library
 * call): the same figures from the same kernels, with the per-block partial sums kept in a static per-GPU
 * scratch array of 512 KiB and added on the device. No counterpart in the reference: it is for callers that
 * cannot allocate, such as a serving or progress-print loop that must not synchronize the device through
 * hipMalloc / hipFree. It is not for HIP graph capture: like decode_error it copies z_host (when given) from
 * pageable host memory and waits on the trainer's stream to copy the totals back. The extent ew x eh may hold
 * at most 2^24 pixels (4096 x 4096); a larger one prints an error and exits, as every other misuse. Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (from several host threads or trainers)
 * race. */
void ntc_trainer_decode_error_noalloc(ntc_trainer* t, const float* z_host, int ew, int eh, double* tex_mse, double* weighted);
/* The figures of the reference's progress line (main.cpp:4155-4212) computed on the device, without downloading
 * the model (the reference's --cuda print path downloads the latent and the weights at every print):
 *   bitrate_stats (main.cpp:2273-2352) as a progress print runs it, the order-0 figure standing in for the
 *   (up, left) context estimate (main.cpp:4171), at --qbits qbits; q_*: mse_of (main.cpp:1764-1788, extent ew x eh,
 *   0 = the whole image) of the decode of the quantized latent it returns; lat_*: latent_stats (main.cpp:2211-2216)
 *   of each level of the shadow; dct_*: with a live --dct-q level 0, dct_analyze (main.cpp:1080-1208) with the code
 *   grid's context estimate, as the line's token group calls it (main.cpp:4180-4190). No counterpart in the
 *   reference's backend. The bitrate figures equal the host computation bit for bit, except that a live DCT
 *   plane's token bits (and dct_analyze's per-class sums) add the same terms per histogram bin instead of per
 *   token (within 1e-13 relative). */
typedef struct ntc_print_stats {
    double bpp_fp32, bpp_q8, bpp_q8_ent, bpp_q8_ctx, bpp_ctx_level0, bpp_est, bits_mlp, bits_raw_latent, bits_header;
    double q_tex_mse[4], q_weighted_mse;
    float lat_mean[NTC_MAX_LEVELS], lat_sd[NTC_MAX_LEVELS], lat_max[NTC_MAX_LEVELS];
    int dct_live;
    double dct_raw[7], dct_h0[7], dct_ctx[7];   /* dc, run, magnitude, sign, end of block, scale code, header */
    double dct_raw_total, dct_h0_total, dct_ctx_total;
    long long dct_nblk, dct_ntok_nz, dct_ntok_eob, dct_nmag_over;
    double dct_nz_mean, dct_lnz_mean, dct_eob_only_frac;
} ntc_print_stats;
void ntc_trainer_print_stats(ntc_trainer* t, int qbits, int ew, int eh, ntc_print_stats* out);
/* The decode of the current model rounded to 8 bits as the reference's save_png and ntc_decode write it
 * (lround of the [0, 1]-clamped value times 255): W*H*nout bytes, interleaved per pixel. No counterpart in
 * the reference's backend (its decoder is the host program ntc_decode.cpp). */
void ntc_trainer_decode_rgb8(ntc_trainer* t, uint8_t* out);

/* Trainer::mlp_step / mlp_step_fd / reset_mlp_adam / mlp_stats (cuda/ntc_cuda.h:110-115) */
void ntc_trainer_mlp_step(ntc_trainer* t, int it, float sigma, float lr, int N, int M);
void ntc_trainer_mlp_step_fd(ntc_trainer* t, int it, float h, float lr, int M);
void ntc_trainer_reset_mlp_adam(ntc_trainer* t);
void ntc_trainer_mlp_stats(ntc_trainer* t, double* batch_loss, double* diff_std);

/* Trainer::lat_step / qat_search / decode_full (cuda/ntc_cuda.h:118-123); z_host may be NULL */
void ntc_trainer_lat_step(ntc_trainer* t, int it, float sigma, float lr, int K);
void ntc_trainer_qat_search(ntc_trainer* t);
void ntc_trainer_decode_full(ntc_trainer* t, const float* z_host, float* img);

/* Trainer::debug_last_batch / debug_last_dl / debug_last_zgrad (cuda/ntc_cuda.h:127-129):
 * copy at most cap values, return how many the trainer holds */
size_t ntc_trainer_debug_last_batch(const ntc_trainer* t, int* bidx, size_t cap);
size_t ntc_trainer_debug_last_dl(const ntc_trainer* t, double* dl, size_t cap);
size_t ntc_trainer_debug_last_zgrad(const ntc_trainer* t, float* g, size_t cap);

/* ---- Instrumentation and verification helpers. No counterpart in the reference: they serve the
 * parity tests and the benchmark, and change no trainer state. ---- */
/* sizeof of a descriptor as this library was compiled ("ntc_model_desc", "ntc_qes_desc", "ntc_dct_desc",
 * "ntc_level_desc"), 0 for an unknown name: lets a binding check its mirror of the layouts */
size_t ntc_abi_sizeof(const char* name);
/* the member losses of the last ES step (pair i: member + is w + sigma eps_i, member - is w - sigma eps_i),
 * or for a central-difference step the losses at w_j + h and w_j - h; returns the pair count */
size_t ntc_trainer_debug_last_losses(const ntc_trainer* t, double* lplus, double* lminus, size_t cap);
/* the MLP weight gradient of the last ES or central-difference step (before Adam), P floats */
size_t ntc_trainer_debug_last_wgrad(const ntc_trainer* t, float* g, size_t cap);
/* the per-pixel loss differences (l+ - l-) / (3 wsum W H) of the last latent ES step, K x W*H floats
 * (pair-major); returns K * W * H, 0 before the first latent step */
size_t ntc_trainer_debug_last_dpix(const ntc_trainer* t, float* d, size_t cap);
long long ntc_trainer_nparams(const ntc_trainer* t);
long long ntc_trainer_nz(const ntc_trainer* t);
void* ntc_trainer_stream(const ntc_trainer* t);        /* the hipStream_t every launch of this trainer uses */
void ntc_trainer_synchronize(ntc_trainer* t);
/* Per-kernel device time with HIP events recorded on the trainer's stream around each launch
 * of the named kernel family ("pop_eval", "lat_pair", "qat_search", ...). */
void ntc_trainer_set_profiling(ntc_trainer* t, int on);
/* restrict the events to the comma-separated kernel families in names (null or "" = every family): each
 * event pair costs the stream a few microseconds */
void ntc_trainer_set_profiling_only(ntc_trainer* t, const char* names);
/* time one launch in n of each family (n <= 1: every launch), counted from the last ntc_trainer_set_profiling(t, 1):
 * a timed launch costs the stream several microseconds around it, so sampling keeps a timed run's own pace */
void ntc_trainer_set_profiling_every(ntc_trainer* t, int n);
int ntc_trainer_kernel_time(ntc_trainer* t, const char* name, double* total_ms, long long* launches);
// 1 if the stage ("pop_eval": the ES and central-difference populations, "lat_pair", "qat_search") runs on
// the FP32 matrix cores for this model, else 0; "pop_pair": 1 if its ES steps with the pairs and minibatch sized at
// init take a population kernel that shares a pair's first layer (k_pop_pair, or k_pop_pair_own for the pixel-per-lane
// shapes); "pop_pair_own": 1 if that kernel is k_pop_pair_own
int ntc_trainer_on_matrix_cores(ntc_trainer* t, const char* stage);
/* on = 0: every stage of this trainer runs on the VALU kernels from the next call on (the matrix-core
 * kernels' parity and speed are then measured against them); on = 1 (the default): the matrix cores
 * take every stage whose shape they pay off for */
void ntc_trainer_set_matrix_cores(ntc_trainer* t, int on);
/* pairs > 0: every latent step of this trainer runs its pairs in groups of at most `pairs` (the Gaussians and
 * per-pixel differences of one group at a time; the results are the same bit for bit); 0 (the default): groups
 * as large as 1 GiB of those buffers holds. ntc_trainer_debug_last_dpix then returns the last group's pairs. */
void ntc_trainer_set_lat_group(ntc_trainer* t, int pairs);
/* Compiles, with hipRTC and without loading it (no device needed), the kernel set that a trainer
 * specialises at init for a model whose shape the library does not list (its hidden layers all one
 * width); arch e.g. "gfx950". Returns 1, or 0 with the compiler's log in why. seconds: the compile time. */
int ntc_jit_compile_check(const ntc_model_desc* d, const char* arch, double* seconds, char* why, size_t why_cap);
/* the device's Gaussian draws for indices index0 .. index0 + n - 1 of one (seed, stream, step, pair) */
void ntc_trainer_debug_gauss(ntc_trainer* t, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index0, size_t n,
                             float* out);
/* The integer histograms behind the last ntc_trainer_print_stats: bitrate (returned count) = for each level l (a live
 * --dct-q level 0 skipped) and channel c, 2^bits(l, c) quantization-index bins, then for l >= 1 as many bins of the
 * DPCM residual of bpp_est; lohi[l * 64 + c][2] = the least and greatest value of the channel (its post-hoc scale);
 * dct (*n_dct values) = per channel run[65] mag[257] ctx_run[64 x 65] ctx_mag[64 x 257] ctxr[64] ctxm[64] dcres[4097]
 * code[16] code_tri[16 x 16 x 16] code_pair[16 x 16] nrun neob nsign, then sum_nz sum_lnz n_lnz eob_only nmag_over.
 * Copies at most the capacities given (lohi: 3 x 64 x 2 floats). */
size_t ntc_trainer_debug_print_counts(const ntc_trainer* t, long long* bitrate, size_t cap_b, float* lohi, long long* dct,
                                      size_t cap_d, size_t* n_dct);
/* runs a plain device copy of n floats (n a multiple of 4) reps times on the trainer's stream:
 * the known-size reference that converts a profile's memory counters into bytes */
void ntc_trainer_debug_copy_calibration(ntc_trainer* t, size_t n, int reps);
/* the device's copy of the two Gaussian factors for 24-bit draws k0 .. k0 + n - 1:
 * rad[k] = sqrtf(-2 logf((k + 1) / 2^24)), cosv[k] = cosf(2 pi k / 2^24) */
void ntc_trainer_debug_noise_factors(ntc_trainer* t, uint32_t k0, size_t n, float* rad, float* cosv);
/* device allocations (hipMalloc) and releases (hipFree) this library has made in the process so far, in *allocs and
 * *frees: read around a call, they show whether it allocated */
void ntc_debug_device_allocations(long long* allocs, long long* frees);

#ifdef __cplusplus
}
#endif
