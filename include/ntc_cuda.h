// Drop-in interface of the MI355X (gfx950) ES training backend.
//
// Declaration-compatible with the reference's cuda/ntc_cuda.h (richgel999/neural_block_textures):
// the namespace, the envelope constants, the five descriptor structs (field names, order, types
// and defaults) and every Trainer method keep their names and meaning, so the reference's
// main.cpp compiles against this header unchanged and links against libntc_hip.so in place of
// the CUDA static library. The name "ntc_cuda" is kept only because main.cpp
// spells it; nothing behind it uses CUDA. Plain C++: no HIP types leak into this header.
//
// Reference: cuda/ntc_cuda.h:14-20 (constants), :23 (PosKindDev), :25-52 (LevelDesc, PosDesc,
// ModelDesc), :57-63 (QesDesc), :68-76 (DctDesc), :78-132 (Trainer).
#pragma once
#include <stdint.h>
#include <stddef.h>
#include <string>
#include <vector>

struct ntc_print_stats;   // the progress line's figures (include/ntc_hip.h)

namespace ntc_cuda {

// Envelope (cuda/ntc_cuda.h:14-20)
static const int MAX_LEVELS = 3;    // latent levels
static const int MAX_POS = 16;      // positional feature generators
static const int MAX_OUT = 12;      // MLP outputs: 3 channels x up to 4 textures
static const int MAX_HIDDEN = 8;    // hidden layers
static const int MAX_CH = 16;       // level-0 channels with a per-channel --qat depth
static const int MAX_QES_CH = 64;   // channels of a --qes level
static const int MAX_DCT_CH = 4;    // channels of a --dct-q level 0

// Positional feature kinds, in main.cpp's PosKind order (cuda/ntc_cuda.h:23)
enum PosKindDev { PK_UV, PK_LV1LOCAL };

struct LevelDesc { int W = 0, H = 0, C = 0; size_t off = 0; bool nearest = false; };
struct PosDesc { int kind = 0; };

// One model, filled by the caller (main.cpp:3882-3906); cuda/ntc_cuda.h:29-52
struct ModelDesc {
    int W = 0, H = 0;            // image size
    int T = 1;                   // textures; nout = 3 T
    int nlev = 0; LevelDesc lv[MAX_LEVELS];
    int npos = 0; PosDesc pos[MAX_POS];
    int nin = 0, nout = 3;
    int nhidden = 0; int hidden[MAX_HIDDEN];
    float leak = 0.01f;          // leaky-ReLU slope
    bool clamp_out = false;      // clamp(s + 0.5) output instead of the sigmoid
    float cw[MAX_OUT];           // per-output-channel loss weight
    float wsum = 1.0f;
    int qat_bits[MAX_CH];        // --qat depth per level-0 channel, 0 when off
    int qat = 0;                 // largest --qat depth (0 = off)
    const float* qat_grid = nullptr;   // the caller's 9 x 257 grid table, copied verbatim at init
    int qes_bits[MAX_LEVELS] = { 0, 0, 0 };   // --qes depth per level (0 = continuous)
    int dct = 0, dct_C = 0, dct_N = 8, dct_dc_step = 4;   // --dct-q level 0
    int dct_q[MAX_DCT_CH] = { 0, 0, 0, 0 };               // per-channel quality (informational: steps arrive with set_dct)
    const float* dct_basis = nullptr;                     // the caller's 8 x 8 basis bit patterns, copied at init
    const int* dct_zigzag = nullptr;                      // zigzag position -> natural index, copied at init
    int max_pairs = 64;          // largest N mlp_step will be called with
    int max_batch = 4096;        // largest minibatch M
    uint64_t seed = 1;
};

// --qes tables fitted on the host and uploaded by set_qes (cuda/ntc_cuda.h:57-63)
struct QesDesc {
    int bits[MAX_LEVELS];
    int live;
    int frozen;                  // 1: the shadow is clamped to [lo, hi] on every snap
    float lo[MAX_LEVELS][MAX_QES_CH], hi[MAX_LEVELS][MAX_QES_CH], range[MAX_LEVELS][MAX_QES_CH];
    int grid_off[MAX_LEVELS][MAX_QES_CH];
};

// --dct-q level-0 description uploaded by set_dct (cuda/ntc_cuda.h:68-76)
struct DctDesc {
    int live, C, BW, BH, N, dc_step;
    int rate_es, rate_trunc; float rate_scale; float lam_t16[16];   // --dct-lambda parts A / B and their host-computed weights
    int lo_w16;                  // --dct-lambda-lo as round(16 W)
    int deadzone;                // --dct-deadzone
};

// The backend (cuda/ntc_cuda.h:78-132). One host thread drives it; every method is synchronous
// with respect to the host buffers it reads or fills.
class Trainer {
public:
    Trainer();
    ~Trainer();
    bool init(const ModelDesc& d, const float* z, const float* p, const float* target, std::string& why);
    std::string banner() const;

    void upload_model(const float* z, const float* p);
    void download_model(float* z, float* p);
    void set_qes(const QesDesc& q, const float* grid, size_t grid_n);
    void snap_latent();
    void shadow_pull(size_t off, size_t n, float f);
    void download_zq(float* zq);
    void set_dct(const DctDesc& d, const uint8_t* code, const int16_t* sym, const int* step);
    void download_dct(int16_t* sym, uint8_t* code);
    void download_dct_rate(int32_t* bits, int32_t* dbits_last_pair, int* ntrunc, int* nz_before, int* hits, int* evals);

    void mlp_step(int it, float sigma, float lr, int N, int M);
    void mlp_step_fd(int it, float h, float lr, int M);
    void reset_mlp_adam();
    void mlp_stats(double& batch_loss, double& diff_std);

    void lat_step(int it, float sigma, float lr, int K);
    void qat_search();
    void decode_full(const float* z_host, float* img);

    void debug_last_batch(std::vector<int>& bidx) const;
    void debug_last_dl(std::vector<double>& dl) const;
    void debug_last_zgrad(std::vector<float>& g) const;

    // Extensions with no counterpart in the reference's Trainer; each replaces a host stall of main.cpp.
    // The decoder sensitivity probe of a --dct-q level 0 on the device (dct_probe_codes, main.cpp:1001-1032).
    void dct_probe(uint8_t* code, float* gain);
    // Decoder::dct_refit on the device (main.cpp:1672-1680): probe, replace the codes, re-snap level 0.
    void dct_refit(uint8_t* code);
    // mse_of (main.cpp:1764-1788) of the device's decode of its decode buffer, or of z_host (nz floats)
    // as decode_full: per-texture and weighted 8-bit MSE over ew x eh.
    void decode_error(const float* z_host, int ew, int eh, double* tex_mse, double* weighted);
    // The decode rounded to 8 bits as save_png writes it: W * H * nout bytes.
    void decode_rgb8(uint8_t* out);
    // The figures of a progress line on the device (bitrate_stats at --qbits qbits, the error of its quantized
    // latent over ew x eh, latent_stats, dct_analyze; main.cpp:4155-4212), without downloading the model.
    void print_stats(int qbits, int ew, int eh, ::ntc_print_stats* out);

    struct Impl;
    Impl* im;
};

}   // namespace ntc_cuda
