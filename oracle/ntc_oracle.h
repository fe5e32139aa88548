/* CPU oracle for the ES training backend of neural_block_textures.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP kernels are compared
 * against; it is never linked into, loaded by or called from the product library
 * (neural_block_textures_amd/). Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.
 *
 * It restates the reference's CPU path (main.cpp and cuda/ntc_noise.h of
 * richgel999/neural_block_textures) with every floating-point operation written out:
 * products that the reference's host build contracts into a fused multiply-add
 * (GCC's default -ffp-contract=fast with FMA hardware) are explicit fmaf() calls here,
 * everything else is compiled with -ffp-contract=off. Each function names the reference
 * lines it follows.
 *
 * All entry points are extern "C" with plain pointers so tests can bind them with ctypes.
 */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_MAX_LEVELS 3
#define OR_MAX_POS 16
#define OR_MAX_OUT 12
#define OR_MAX_HIDDEN 8
#define OR_MAXH 128

typedef struct OrLevel {
    int W, H, C, nearest;
    long long off;            /* first value of the level in the flat latent vector */
} OrLevel;

typedef struct OrModel {
    int W, H;                 /* image size */
    int nout;                 /* 3 * textures */
    int nlev;
    OrLevel lv[OR_MAX_LEVELS];
    int npos;
    int pos[OR_MAX_POS];      /* 0 = uv, 1 = lv1local */
    int nin;                  /* latent channels + 2 * npos */
    int nhidden;
    int hidden[OR_MAX_HIDDEN];
    float leak;
    int clamp_out;
    float cw[OR_MAX_OUT];
    float wsum;
} OrModel;

/* DCT-coded level 0 state, [block][channel] arrays as in main.cpp DctLevel (main.cpp:709-740). */
typedef struct OrDct {
    int C, BW, BH, dc_step, deadzone, lo_w16;
    float lam_t16[16];
    const int* step;          /* C x 16 x 64 */
    uint8_t* code;            /* BW*BH*C */
    int16_t* sym;             /* BW*BH*C*64 */
} OrDct;

/* ---- counter-based noise (cuda/ntc_noise.h:20-47) ---- */
uint64_t or_mix64(uint64_t x);
uint64_t or_noise_key(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index);
uint32_t or_noise_u32(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index);
uint32_t or_noise_uniform(uint32_t u, uint32_t n);
float or_gauss(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index);
void or_gauss_fill(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index0, long long n, float* out);
/* the two factors of the Gaussian for one 24-bit draw: sqrtf(-2 logf(u1)) and cosf(2 pi u2) */
float or_gauss_radius(uint32_t k1);
float or_gauss_cosine(uint32_t k2);
void or_gauss_factors(uint32_t k0, long long n, float* rad, float* cosv);

/* ---- model geometry and MLP ---- */
long long or_model_nparams(const OrModel* m);
long long or_model_nz(const OrModel* m);
void or_tap(const OrLevel* L, float u, float v, int* x0x1y0y1, float* fxfy);
void or_features(const OrModel* m, const float* z, int px, int py, float* f);
void or_mlp_forward(const OrModel* m, const float* p, const float* in, float* out);
void or_decode_full(const OrModel* m, const float* p, const float* z, float* img);
void or_decode_err(const OrModel* m, const float* p, const float* z, const float* tgt, float* err);
double or_loss_subset(const OrModel* m, const float* p, const float* z, const float* tgt, const int* idx, int n);

/* ---- MLP ES / FD / Adam ---- */
void or_draw_batch(uint64_t seed, int it, int M, int npix, int* idx);
void or_mlp_es_eval(const OrModel* m, const float* p0, const float* z, const float* tgt, uint64_t seed, int it,
                    float sigma, int N, const int* idx, int M, double* dl, double* lsum, double* lp, double* lm);
void or_mlp_es_grad(long long P, int N, uint64_t seed, int it, float sigma, const double* dl, float* grad);
void or_adam(float* theta, const float* g, float* m, float* v, long long n, float lr, int t);
void or_mlp_fd_eval(const OrModel* m, const float* p0, const float* z, const float* tgt, float h,
                    const int* idx, int M, double* dl, double* hh, double* l0);
void or_fd_grad(long long P, const double* dl, const double* hh, float* grad);

/* ---- latent ES (main.cpp:1974-2044 and the rate pass 1935-1952) ----
 * zdec: the decode buffer the pair is built around; the gradient is returned, not applied.
 * active_mask: bit l set = level l is ES-perturbed. dct may be null (no rate term).
 * dpix (nullable): K x W*H per-pixel loss differences (e+ - e-) * inv_px. */
void or_lat_grad(const OrModel* m, const float* p, const float* zdec, const float* zshadow, const float* tgt,
                 uint64_t seed, int step_no, float sigma, int K, unsigned active_mask,
                 const OrDct* dct, float rate_scale, float* grad, float* dpix, int32_t* dbits_last, int* hits);
// the scatter of or_lat_grad alone, from given dpix [K][W*H] and eps [K][nz] (no rate term)
void or_lat_scatter(const OrModel* m, const float* eps, const float* dpix, int K, unsigned active_mask, float sigma,
                    float* grad);

/* ---- --qat (main.cpp:2054-2139) ---- */
void or_qat_grid(float* grid /* 9 x 257 */);
int or_qat_index(float v, int bits);
void or_qat_search(const OrModel* m, const float* p, float* zdec, const float* tgt, const int* ch_bits, const float* grid);

/* ---- --qes (main.cpp:446-495) ---- */
int or_qes_index(float v, float lo, float range, int levels);
void or_qes_fit(const OrLevel* L, const float* z, int bits, float* lo, float* hi, float* range, float* grid);
long long or_qes_snap_level(const OrLevel* L, int bits, const float* lo, const float* hi, const float* range,
                            const float* grid, float* z, float* zq, int clamp);

/* ---- --dct-q (main.cpp:657-1032) ---- */
void or_dct_tables(float* basis /* 64 */, int* zigzag /* 64 */, float* ak /* 16 */);
void or_dct_build_steps(int q, int dc_step, int* out /* 16 x 64 */);
void or_dct_build_steps_scaled(int q, float level_scale, int dc_step, int* out /* 64 */);
float or_dct_quality_scale(int q);
void or_dct_fwd8(const float* w, float* C);
void or_dct_inv8(const float* C, float* w);
int or_dct_quant_dc(float d, int S);
float or_dct_dequant_dc(int q, int S);
int or_dct_quant_ac(float d, int L, int u, int v, int dz);
float or_dct_dequant_ac(int q, int L, int u, int v, int dz);
int or_dct_c_run(int r);
int or_dct_c_mag(int m);
int or_dct_block_bits(const int16_t* sym, int lo16);
int or_dct_quantize_block(const float* Cf, const int* st, int dc_step, float lam16, int lo16, int dz, int with_bits,
                          int16_t* sym, int* ntrunc, int* nz_before);
int or_dct_code_of_gain(double g);
double or_dct_gain_of_code(int k);
void or_dct_clamp_level0(const OrLevel* L0, float* z);
/* snap the whole level 0: shadow clamped in place, symbols written, zq level 0 rebuilt.
 * bits (nullable) receives the proxy bits of every (block, channel); counts[0..2] = ntrunc, nz_before, clamped */
void or_dct_snap_level0(const OrDct* d, const OrLevel* L0, float* z, float* zq, int32_t* bits, long long* counts);
void or_dct_recon_level0(const OrDct* d, const OrLevel* L0, float* zq, int32_t* bits);
void or_dct_probe_codes(const OrModel* m, const float* p, const float* zdec, const OrDct* d, uint8_t* code);
void or_dct_rate_pair(const OrDct* d, const OrLevel* L0, const float* z, const float* eps0, float sg, int32_t* dbits);

/* ---- --dct-shadow-pull (main.cpp:4142-4146): z += f * (zq - z) on n values */
void or_shadow_pull(float* z, const float* zq, long long n, float f);

/* ---- fp16 weight rounding (main.cpp:2427-2481) and post-hoc latent quantization (main.cpp:478-482) ---- */
uint16_t or_f32_to_f16(float f, int* overflow);
float or_f16_to_f32(uint16_t h);
int or_round_fp16(float* p, long long n, long long* changed);
int or_q8_index(float z, float lo, float range, int levels);
float or_q8_value(int k, float lo, float range, int levels);

/* ---- the printed error (mse_of, main.cpp:1764-1788): a and b are W*H*nc (nc = 3 T), w[T], extent ew x eh
 * (0 = whole); tex[T] = SSE_t / (3 ew eh), *weighted = sum_t w_t SSE_t / (3 wsum ew eh), 8-bit rounding ---- */
void or_mse_of(const float* a, const float* b, int W, int H, int nc, const float* w, float wsum, int ew, int eh, double* tex,
               double* weighted);

/* ---- full training driver (main.cpp:4063-4148, --rng hash), for trajectory parity and timing ---- */
typedef struct OrTrainCfg {
    uint64_t seed;
    int mlp_pairs, mlp_batch;
    float mlp_sigma, mlp_lr;
    int lat_pairs;
    float lat_sigma, lat_lr;
    int qat;                  /* 0 = off; bits per level-0 channel in qat_ch */
    int qat_ch[16];
    int fd_from;              /* first FD iteration (iters + 1 = never) */
    float fd_h;
} OrTrainCfg;
typedef struct OrTrainState {
    float* z;                 /* shadow latent, nz */
    float* p;                 /* weights, P */
    float* wm; float* wv; int wt;   /* MLP Adam */
    float* zm; float* zv; int zt;   /* latent Adam */
    int lat_step_no;
} OrTrainState;
/* One iteration it (1-based) of the CPU training loop: MLP ES or FD step, latent step, qat search.
 * tgt is W*H*nout. Returns the MLP step's batch loss. */
double or_train_iter(const OrModel* m, const OrTrainCfg* c, OrTrainState* s, const float* tgt, int it, int iters);

#ifdef __cplusplus
}
#endif

#ifdef __cplusplus
extern "C" {
#endif
/* ---- the progress print's statistics (main.cpp:4155-4212): bitrate_stats (main.cpp:2220-2352, with the
 * order-0 figure standing in for the context estimate as on a progress print), dct_analyze (main.cpp:1049-1208)
 * and latent_stats (main.cpp:2211-2216). */
typedef struct OrPrintIn {
    int qbits;                        /* --qbits: the post-hoc depth of a continuous level */
    int qat; int qat_ch[16];          /* qat > 0: level 0 discrete, qat_ch bits per channel */
    int qes_on;                       /* the model has --qes levels (qes_bits); a continuous one is quantized at its depth */
    int qes_live;                     /* --qes levels trained quantized: indices by qes_index with qes_lo / qes_range */
    int qes_bits[OR_MAX_LEVELS];
    const float* qes_lo;              /* [level][64] */
    const float* qes_range;           /* [level][64] */
    int dct_live; const OrDct* dct; int dc_raw_bits;
    int dct_ctx;                      /* dct_analyze with the code grid's context estimate (g_ctx_stats) */
} OrPrintIn;
typedef struct OrBitrate {
    double bpp_fp32, bpp_q8, bpp_q8_ent, bpp_q8_ctx, bpp_ctx_level0, bpp_est, bits_mlp, bits_raw_latent, bits_header;
} OrBitrate;
typedef struct OrDctStats {
    double raw[7], h0[7], ctx[7];     /* dc, run, mag, sign, eob, code, header */
    double raw_total, h0_total, ctx_total, code_raw, code_h0, code_ctx, header;
    long long nblk, ntok_nz, ntok_eob, nmag_over;
    double nz_mean, lnz_mean, eob_only_frac;
} OrDctStats;
/* bitrate_stats: figures, and zq = the quantized latent it returns (nz floats); P = MLP parameters */
void or_bitrate_stats(const OrModel* m, const OrPrintIn* in, long long P, const float* z, const float* zdec, OrBitrate* out, float* zq);
/* dct_analyze of all channels */
void or_dct_analyze(const OrDct* d, int dc_raw_bits, int ctx, OrDctStats* out);
/* latent_stats of level l of z */
void or_latent_stats(const OrModel* m, int l, const float* z, float* mean, float* sd, float* mx);

/* The integer histograms the figures above are sums over (the device path fills the same layout):
 *   bitrate: for each level l (a live DCT level 0 skipped), each channel c, with nb = 2^bits(l, c): nb index bins, then for
 *            l >= 1 nb bins of the DPCM residual (cur - pred) & (nb - 1) of bpp_est; lohi[l][c][2] = the channel's min and
 *            max (continuous levels; the post-hoc scale)
 *   dct, per channel: run[65] mag[257] ctx_run[64 x 65] ctx_mag[64 x 257] ctxr[64] ctxm[64] dcres[4097] code[16]
 *            code_tri[16 x 16 x 16] (up, left, code) code_pair[16 x 16] (up, left) nrun neob nsign; then over all channels
 *            sum_nz sum_lnz n_lnz eob_only nmag_over
 * or_print_counts_size returns both sizes; or_print_counts fills them (lohi: 3 x 64 x 2 floats). */
#define OR_DCT_COUNTS_PER_CH (65 + 257 + 64 * 65 + 64 * 257 + 64 + 64 + 4097 + 16 + 4096 + 256 + 3)
#define OR_DCT_COUNTS_TAIL 5
void or_print_counts_size(const OrModel* m, const OrPrintIn* in, long long* n_bitrate, long long* n_dct);
void or_print_counts(const OrModel* m, const OrPrintIn* in, const float* z, const float* zdec, long long* bitrate, float* lohi,
                     long long* dct);
/* The widest x86-64 level the host CPU and OS support, by cpuid: 4 (AVX-512 F/BW/CD/DQ/VL), 3 (AVX2, FMA,
 * BMI2), else 1. Picks the reference build the CPU baseline loads. */
int or_host_isa_level(void);
#ifdef __cplusplus
}
#endif
