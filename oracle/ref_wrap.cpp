// Reference build: the reference's own CPU path, compiled from main.cpp where it lies under the
// reference tree (never copied), with extern "C" entry points that mirror the oracle's so tests
// and the golden-vector script can run the two side by side.
//
// TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile into oracle/_ref/ (git-ignored) from
// $(REF)/main.cpp. Two builds: libntc_ref.so with GCC's default floating point (FMA contraction
// on, no reassociation) for golden vectors, and libntc_ref_fast.so with the reference's own
// CMake flags (-O3 -ffast-math, CMakeLists.txt:24) for the CPU-baseline timing.
//
// The only addition to the reference's text: libstdc++ 11 declares fabsf / floorf in the global
// namespace but not in std, and main.cpp:809-812 call std::fabsf / std::floorf, so the two
// using-declarations below make them visible there. Everything else is main.cpp unmodified.
#include <cmath>
namespace std { using ::fabsf; using ::floorf; }

#define main ntc_reference_main
#include "main.cpp"
#undef main

#include "ntc_oracle.h"

namespace {

// A Decoder built from the oracle's model description (the fields main.cpp:3470-3564 fills).
struct RefModel {
    Options o;
    Decoder D;
    Image target;
};

void fill_decoder(RefModel& R, const OrModel& m, const float* z, const float* p, const float* tgt) {
    Decoder& D = R.D;
    D.opt = &R.o;
    R.o.clamp_out = m.clamp_out != 0;
    std::string spec;
    for (int q = 0; q < m.npos; q++) spec += std::string(q ? "," : "") + (m.pos[q] == 0 ? "uv" : "lv1local");
    D.pos.parse(spec.empty() ? "none" : spec);
    D.W = m.W; D.H = m.H;
    D.lat = LatentSet();
    for (int l = 0; l < m.nlev; l++) D.lat.add(m.lv[l].W, m.lv[l].H, m.lv[l].C, m.lv[l].nearest != 0);
    if (z) memcpy(D.lat.z.data(), z, D.lat.z.size() * sizeof(float));
    D.mlp.nout = m.nout;
    D.mlp.nin = D.nin();
    D.mlp.hidden.assign(m.hidden, m.hidden + m.nhidden);
    D.mlp.leak = m.leak;
    D.mlp.p.assign((size_t)MLP::count(D.mlp.widths()), 0.0f);
    if (p) memcpy(D.mlp.p.data(), p, D.mlp.p.size() * sizeof(float));
    D.cw.assign(m.cw, m.cw + m.nout);
    D.wsum = m.wsum;
    D.qes.assign(m.nlev, QesLevel());
    R.target.w = m.W; R.target.h = m.H; R.target.nc = m.nout;
    if (tgt) R.target.rgb.assign(tgt, tgt + (size_t)m.W * m.H * m.nout);
}

}   // namespace

extern "C" {

float ref_gauss(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index) { return ntc_gauss(seed, stream, step, pair, index); }
uint32_t ref_noise_u32(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index) { return ntc_noise_u32(seed, stream, step, pair, index); }
uint32_t ref_noise_uniform(uint32_t u, uint32_t n) { return ntc_noise_uniform(u, n); }

void ref_features(const OrModel* m, const float* z, int px, int py, float* f) {
    RefModel R; fill_decoder(R, *m, z, nullptr, nullptr);
    R.D.features(R.D.lat.z.data(), px, py, f);
}
void ref_mlp_forward(const OrModel* m, const float* p, const float* in, float* out) {
    RefModel R; fill_decoder(R, *m, nullptr, p, nullptr);
    mlp_forward(R.D.mlp, R.D.mlp.p.data(), in, out, m->clamp_out != 0);
}
void ref_decode_full(const OrModel* m, const float* p, const float* z, float* img) {
    RefModel R; fill_decoder(R, *m, z, p, nullptr);
    Image out; R.D.decode_full(R.D.mlp.p.data(), R.D.lat.z.data(), out);
    memcpy(img, out.rgb.data(), out.rgb.size() * sizeof(float));
}
void ref_decode_err(const OrModel* m, const float* p, const float* z, const float* tgt, float* err) {
    RefModel R; fill_decoder(R, *m, z, p, tgt);
    std::vector<float> e; R.D.decode_err(R.D.mlp.p.data(), R.D.lat.z.data(), R.target, e);
    memcpy(err, e.data(), e.size() * sizeof(float));
}
double ref_loss_subset(const OrModel* m, const float* p, const float* z, const float* tgt, const int* idx, int n) {
    RefModel R; fill_decoder(R, *m, z, p, tgt);
    std::vector<int> ix(idx, idx + n);
    return R.D.loss_subset(R.D.mlp.p.data(), R.D.lat.z.data(), R.target, ix);
}

// MlpTrainer::step (--rng hash): p, Adam m/v/t updated in place; grad (nullable) = the gradient
// before Adam; returns the mean pair loss, *dstd the spread of the pair differences.
double ref_mlp_step(const OrModel* m, float* p, const float* z, const float* tgt, uint64_t seed, int it, float sigma,
                    float lr, int N, int M, float* am, float* av, int* at, float* grad, double* dstd) {
    RefModel R; fill_decoder(R, *m, z, p, tgt);
    R.o.rng_hash = true; R.o.seed = (unsigned)seed; R.o.mlp_pairs = N; R.o.mlp_batch = M; R.o.mlp_sigma = sigma; R.o.mlp_lr = lr;
    MlpTrainer mt; mt.init(R.D.mlp.size());
    const size_t P = R.D.mlp.size();
    mt.adam.m.assign(am, am + P); mt.adam.v.assign(av, av + P); mt.adam.t = *at;
    mt.cur_it = it;
    std::mt19937 rng(1);
    double ds = 0;
    const double l = mt.step(R.D, R.target, rng, R.o, ds);
    memcpy(p, R.D.mlp.p.data(), P * sizeof(float));
    memcpy(am, mt.adam.m.data(), P * sizeof(float)); memcpy(av, mt.adam.v.data(), P * sizeof(float)); *at = mt.adam.t;
    if (grad) memcpy(grad, mt.grad.data(), P * sizeof(float));
    if (dstd) *dstd = ds;
    return l;
}
// MlpTrainer::step_fd (--rng hash minibatch)
double ref_mlp_step_fd(const OrModel* m, float* p, const float* z, const float* tgt, uint64_t seed, int it, float h,
                       float lr, int M, float* am, float* av, int* at, float* grad, double* fdrms) {
    RefModel R; fill_decoder(R, *m, z, p, tgt);
    R.o.rng_hash = true; R.o.seed = (unsigned)seed; R.o.mlp_batch = M; R.o.mlp_fd_h = h; R.o.mlp_lr = lr;
    MlpTrainer mt; mt.init(R.D.mlp.size());
    const size_t P = R.D.mlp.size();
    mt.adam.m.assign(am, am + P); mt.adam.v.assign(av, av + P); mt.adam.t = *at;
    mt.cur_it = it;
    std::mt19937 rng(1);
    double ds = 0;
    const double l = mt.step_fd(R.D, R.target, rng, R.o, ds);
    memcpy(p, R.D.mlp.p.data(), P * sizeof(float));
    memcpy(am, mt.adam.m.data(), P * sizeof(float)); memcpy(av, mt.adam.v.data(), P * sizeof(float)); *at = mt.adam.t;
    if (grad) memcpy(grad, mt.grad.data(), P * sizeof(float));
    if (fdrms) *fdrms = ds;
    return l;
}
void ref_draw_batch(uint64_t seed, int it, int M, const OrModel* m, int* idx) {
    RefModel R; fill_decoder(R, *m, nullptr, nullptr, nullptr);
    R.o.rng_hash = true; R.o.seed = (unsigned)seed; R.o.mlp_batch = M;
    MlpTrainer mt; mt.cur_it = it;
    std::mt19937 rng(1);
    mt.draw_batch(R.D, rng, R.o);
    memcpy(idx, mt.batch.data(), (size_t)M * sizeof(int));
}

// LatentTrainer::step (--rng hash, no --qes / --dct-q): z (the shadow, also the decode buffer)
// updated in place by Adam; grad = the gradient before Adam. qat > 0 freezes level 0.
void ref_lat_step(const OrModel* m, const float* p, float* z, const float* tgt, uint64_t seed, int step_no, float sigma,
                  float lr, int K, int qat, float* am, float* av, int* at, float* grad) {
    RefModel R; fill_decoder(R, *m, z, p, tgt);
    R.o.rng_hash = true; R.o.seed = (unsigned)seed; R.o.lat_pairs = K; R.o.lat_sigma = sigma; R.o.lat_lr = lr; R.o.qat = qat;
    LatentTrainer lt; lt.init(R.D.lat.size());
    const size_t n = R.D.lat.size();
    lt.adam.m.assign(am, am + n); lt.adam.v.assign(av, av + n); lt.adam.t = *at;
    lt.step_no = step_no;
    std::mt19937 rng(1);
    lt.step(R.D, R.target, rng, R.o);
    memcpy(z, R.D.lat.z.data(), n * sizeof(float));
    memcpy(am, lt.adam.m.data(), n * sizeof(float)); memcpy(av, lt.adam.v.data(), n * sizeof(float)); *at = lt.adam.t;
    if (grad) memcpy(grad, lt.grad.data(), n * sizeof(float));
}

// qat_search on level 0 of z (the decode buffer; no --qes level)
void ref_qat_search(const OrModel* m, const float* p, float* z, const float* tgt, const int* ch_bits) {
    RefModel R; fill_decoder(R, *m, z, p, tgt);
    qat_init_grid();
    std::vector<int> bits(ch_bits, ch_bits + m->lv[0].C);
    R.D.qat_bits = *std::max_element(bits.begin(), bits.end()); R.D.qat_ch = bits;
    qat_search(R.D, R.target, bits);
    memcpy(z, R.D.lat.z.data(), R.D.lat.z.size() * sizeof(float));
}
void ref_qat_grid(float* grid) { qat_init_grid(); memcpy(grid, QAT_GRID, sizeof(QAT_GRID)); }
int ref_qat_index(float v, int bits) { return qat_index(v, bits); }

int ref_qes_index(float v, float lo, float range, int levels) { return qes_index(v, lo, range, levels); }
void ref_qes_fit(const OrLevel* L, const float* z, int bits, float* lo, float* hi, float* range, float* grid) {
    Latent Lv; Lv.W = L->W; Lv.H = L->H; Lv.C = L->C;
    QesLevel Q; Q.bits = bits;
    qes_fit(Q, Lv, z);
    memcpy(lo, Q.lo.data(), L->C * sizeof(float)); memcpy(hi, Q.hi.data(), L->C * sizeof(float));
    memcpy(range, Q.range.data(), L->C * sizeof(float)); memcpy(grid, Q.grid.data(), Q.grid.size() * sizeof(float));
}
long long ref_qes_snap_level(const OrLevel* L, int bits, const float* lo, const float* hi, const float* range,
                             const float* grid, float* z, float* zq, int clamp) {
    Latent Lv; Lv.W = L->W; Lv.H = L->H; Lv.C = L->C;
    QesLevel Q; Q.bits = bits;
    Q.lo.assign(lo, lo + L->C); Q.hi.assign(hi, hi + L->C); Q.range.assign(range, range + L->C);
    Q.grid.assign(grid, grid + (size_t)L->C * (1 << bits));
    return (long long)qes_snap_level(Q, Lv, z, zq, clamp != 0);
}

// ---- DCT
void ref_dct_tables(float* basis, int* zigzag, float* ak) {
    dct_init_tables();
    if (basis) memcpy(basis, DCT_BASIS, sizeof(DCT_BASIS));
    if (zigzag) memcpy(zigzag, DCT_ZIGZAG, sizeof(DCT_ZIGZAG));
    if (ak) memcpy(ak, DCT_AK, sizeof(DCT_AK));
}
int ref_dct_selftest() { return dct_selftest(); }
void ref_dct_build_steps(int q, int dc_step, int* out) { dct_init_tables(); dct_build_steps(q, 8, dc_step, out); }
void ref_dct_fwd8(const float* w, float* C) { dct_init_tables(); dct_fwd8(w, C); }
void ref_dct_inv8(const float* C, float* w) { dct_init_tables(); dct_inv8(C, w); }
int ref_dct_quant_ac(float d, int L, int u, int v, int dz) { return dct_quant_ac(d, L, u, v, dz != 0); }
float ref_dct_dequant_ac(int q, int L, int u, int v, int dz) { return dct_dequant_ac(q, L, u, v, dz != 0); }
int ref_dct_quant_dc(float d, int S) { return dct_quant_dc(d, S); }
int ref_dct_block_bits(const int16_t* sym, int lo16) { dct_init_tables(); return dct_block_bits(sym, lo16); }
int ref_dct_quantize_block(const float* Cf, const int* st, int dc_step, float lam16, int lo16, int dz, int with_bits,
                           int16_t* sym, int* ntrunc, int* nz_before) {
    dct_init_tables();
    return dct_quantize_block(Cf, st, dc_step, lam16, lo16, dz != 0, with_bits != 0, sym, ntrunc, nz_before);
}
int ref_dct_code_of_gain(double g) { return dct_code_of_gain(g); }

namespace {
DctLevel dct_level_of(const OrDct* d) {
    dct_init_tables();
    DctLevel Q;
    Q.on = true; Q.live = true; Q.N = 8; Q.dc_step = d->dc_step; Q.deadzone = d->deadzone != 0;
    Q.BW = d->BW; Q.BH = d->BH; Q.C = d->C; Q.lo_w16 = d->lo_w16;
    Q.sym.assign(d->sym, d->sym + Q.nblk() * Q.C * 64);
    Q.code.assign(d->code, d->code + Q.nblk() * Q.C);
    Q.step.assign(d->step, d->step + (size_t)Q.C * 16 * 64);
    bool lam = false;
    for (int k = 0; k < 16; k++) { Q.lam_t16[k] = d->lam_t16[k]; if (d->lam_t16[k] > 0.0f) lam = true; }
    Q.lambda = lam ? 1.0f : 0.0f;   // only its sign is read (the bits fill of dct_recon_block)
    Q.bits.assign(Q.nblk() * Q.C, 0);
    return Q;
}
}
void ref_dct_snap_level0(const OrDct* d, const OrLevel* L0, float* z, float* zq, int32_t* bits, long long* counts) {
    DctLevel Q = dct_level_of(d);
    Latent L; L.W = L0->W; L.H = L0->H; L.C = L0->C;
    dct_snap_level0(Q, L, z, zq);
    memcpy(d->sym, Q.sym.data(), Q.sym.size() * sizeof(int16_t));
    if (bits) memcpy(bits, Q.bits.data(), Q.bits.size() * sizeof(int32_t));
    if (counts) { counts[0] = (long long)Q.last_truncated; counts[1] = (long long)Q.last_nz_before; counts[2] = (long long)Q.last_clamped; }
}
void ref_dct_recon_level0(const OrDct* d, const OrLevel* L0, float* zq, int32_t* bits) {
    DctLevel Q = dct_level_of(d);
    Latent L; L.W = L0->W; L.H = L0->H; L.C = L0->C;
    dct_recon_level0(Q, L, zq);
    if (bits) memcpy(bits, Q.bits.data(), Q.bits.size() * sizeof(int32_t));
}
void ref_dct_probe_codes(const OrModel* m, const float* p, const float* zdec, const OrDct* d, uint8_t* code) {
    RefModel R; fill_decoder(R, *m, zdec, p, nullptr);
    DctLevel Q = dct_level_of(d);
    std::vector<uint8_t> out;
    const float* zz = R.D.lat.z.data();
    dct_probe_codes(R.D.mlp, m->clamp_out != 0, R.D.cw, R.D.wsum, Q, [&](int px, int py, float* f) { R.D.features(zz, px, py, f); }, out);
    memcpy(code, out.data(), out.size());
}
void ref_dct_rate_pair(const OrDct* d, const OrLevel* L0, const float* z, const float* eps0, float sg, int32_t* dbits) {
    DctLevel Q = dct_level_of(d);
    Latent L; L.W = L0->W; L.H = L0->H; L.C = L0->C;
    const long long nb = (long long)Q.nblk();
    for (long long b = 0; b < nb; b++)
        for (int c = 0; c < Q.C; c++)
            dbits[(size_t)b * Q.C + c] = dct_rate_block(Q, L, (size_t)b, c, z, eps0, sg, 1.0f) - dct_rate_block(Q, L, (size_t)b, c, z, eps0, sg, -1.0f);
}

// ---- the printed error
void ref_mse_of(const float* a, const float* b, int W, int H, int nc, const float* w, float wsum, int ew, int eh, double* tex,
                double* weighted) {
    Image A, B;
    A.w = B.w = W; A.h = B.h = H; A.nc = B.nc = nc;
    A.rgb.assign(a, a + (size_t)W * H * nc); B.rgb.assign(b, b + (size_t)W * H * nc);
    const Mse m = mse_of(A, B, std::vector<float>(w, w + nc / 3), wsum, ew, eh);
    for (int t = 0; t < nc / 3; t++) tex[t] = m.tex[t];
    *weighted = m.weighted;
}

// ---- the progress print's statistics: the reference's own bitrate_stats (with g_ctx_stats off, as a progress
// print runs it, main.cpp:4171), dct_analyze (g_ctx_stats as asked) and latent_stats
namespace {
void print_decoder(RefModel& R, const OrModel* m, const OrPrintIn* in, const float* z, const float* zdec, long long P) {
    std::vector<float> p((size_t)P, 0.0f);
    fill_decoder(R, *m, z, p.data(), nullptr);
    Decoder& D = R.D;
    if (in->qat > 0) {
        qat_init_grid();
        D.qat_ch.assign(in->qat_ch, in->qat_ch + m->lv[0].C);
        D.qat_bits = *std::max_element(D.qat_ch.begin(), D.qat_ch.end());
    }
    D.qes_on = in->qes_on != 0;
    D.qes_live = in->qes_live != 0;
    for (int l = 0; l < m->nlev; l++) {
        D.qes[l].bits = in->qes_bits[l];
        if (in->qes_live && in->qes_bits[l] > 0) {
            const int C = m->lv[l].C;
            D.qes[l].lo.assign(in->qes_lo + l * 64, in->qes_lo + l * 64 + C);
            D.qes[l].range.assign(in->qes_range + l * 64, in->qes_range + l * 64 + C);
            D.qes[l].hi.assign(C, 0.0f);
        }
    }
    if (in->dct_live) {
        D.dct = dct_level_of(in->dct);
        D.dct.dc_raw_bits = in->dc_raw_bits;
    }
    D.zq.assign(zdec, zdec + D.lat.z.size());
}
}   // namespace
void ref_bitrate_stats(const OrModel* m, const OrPrintIn* in, long long P, const float* z, const float* zdec, OrBitrate* out, float* zq) {
    RefModel R; print_decoder(R, m, in, z, zdec, P);
    std::vector<float> q;
    g_ctx_stats = false;
    const BitrateStats b = bitrate_stats(R.D, in->qbits, q);
    g_ctx_stats = true;
    out->bpp_fp32 = b.bpp_fp32; out->bpp_q8 = b.bpp_q8; out->bpp_q8_ent = b.bpp_q8_ent; out->bpp_q8_ctx = b.bpp_q8_ctx;
    out->bpp_ctx_level0 = b.bpp_ctx_level0; out->bpp_est = b.bpp_est; out->bits_mlp = b.bits_mlp;
    out->bits_raw_latent = b.bits_raw_latent; out->bits_header = b.bits_header;
    memcpy(zq, q.data(), q.size() * sizeof(float));
}
void ref_dct_analyze(const OrDct* d, int dc_raw_bits, int ctx, OrDctStats* out) {
    DctLevel Q = dct_level_of(d);
    Q.dc_raw_bits = dc_raw_bits;
    g_ctx_stats = ctx != 0;
    const DctStats S = dct_analyze(Q);
    g_ctx_stats = true;
    memset(out, 0, sizeof(*out));
    for (int k = 0; k < 7; k++) { out->raw[k] = S.raw[k]; out->h0[k] = S.h0[k]; out->ctx[k] = S.ctx[k]; }
    out->raw_total = S.raw_total; out->h0_total = S.h0_total; out->ctx_total = S.ctx_total;
    out->code_raw = S.code_raw; out->code_h0 = S.code_h0; out->code_ctx = S.code_ctx; out->header = S.header;
    out->nblk = (long long)S.nblk; out->ntok_nz = (long long)S.ntok_nz; out->ntok_eob = (long long)S.ntok_eob;
    out->nmag_over = (long long)S.nmag_over;
    out->nz_mean = S.nz_mean; out->lnz_mean = S.lnz_mean; out->eob_only_frac = S.eob_only_frac;
}
void ref_latent_stats(const OrModel* m, int l, const float* z, float* mean, float* sd, float* mx) {
    RefModel R; fill_decoder(R, *m, z, nullptr, nullptr);
    latent_stats(R.D.lat.lv[l], R.D.lat.level(l), *mean, *sd, *mx);
}

// ---- fp16 and post-hoc quantization
int ref_ntcb_selfcheck() { return ntcb_selfcheck() ? 1 : 0; }
uint16_t ref_f32_to_f16(float f, int* overflow) { bool ov = false; const uint16_t h = ntcb_f32_to_f16(f, &ov); *overflow = ov ? 1 : 0; return h; }
float ref_f16_to_f32(uint16_t h) { return ntcb_f16_to_f32(h); }
int ref_q8_index(float z, float lo, float range, int levels) { return q8_index(z, lo, range, levels); }

// ---- the training loop (main.cpp:4063-4148, CPU branch, --rng hash): a persistent context so a
// sample of iterations can be timed with the trainers' own state.
struct RefTrain {
    RefModel R;
    MlpTrainer mt;
    LatentTrainer lt;
    std::mt19937 rng{ 1 };
    int fd_from = 0;
    float shadow_pull = 0.0f;   // --dct-shadow-pull (the reference's default 0.01 with a DCT level)
    int dct_start_it = 0;       // the DCT switch (main.cpp:3804): 0 = the plane is live from the start
};
void* ref_train_create(const OrModel* m, const OrTrainCfg* c, const float* z, const float* p, const float* tgt) {
    RefTrain* T = new RefTrain;
    fill_decoder(T->R, *m, z, p, tgt);
    Options& o = T->R.o;
    o.rng_hash = true; o.seed = (unsigned)c->seed;
    o.mlp_pairs = c->mlp_pairs; o.mlp_batch = c->mlp_batch; o.mlp_sigma = c->mlp_sigma; o.mlp_lr = c->mlp_lr;
    o.lat_pairs = c->lat_pairs; o.lat_sigma = c->lat_sigma; o.lat_lr = c->lat_lr;
    o.qat = c->qat; o.qat_ch.assign(c->qat_ch, c->qat_ch + m->lv[0].C); o.mlp_fd_h = c->fd_h;
    if (o.qat > 0) { qat_init_grid(); T->R.D.qat_bits = o.qat; T->R.D.qat_ch = o.qat_ch; }
    T->fd_from = c->fd_from;
    T->mt.init(T->R.D.mlp.size());
    T->lt.init(T->R.D.lat.size());
    return T;
}
// The same loop with a live DCT-coded level 0 (codes and steps given): every decode reads the snapped
// plane, the latent step adds the rate pass with --dct-lambda part A and re-snaps (main.cpp:1638-1648, 1972).
void* ref_train_create_dct(const OrModel* m, const OrTrainCfg* c, const float* z, const float* p, const float* tgt,
                           const OrDct* d, float lambda, int rate_es, int rate_trunc) {
    RefTrain* T = (RefTrain*)ref_train_create(m, c, z, p, tgt);
    Decoder& D = T->R.D;
    D.dct = dct_level_of(d);
    D.dct.lambda = lambda; D.dct.rate_es = rate_es != 0; D.dct.rate_trunc = rate_trunc != 0;
    D.zq.assign(D.lat.z.size(), 0.0f);
    D.qes_refresh();
    T->shadow_pull = 0.01f;   // the default --dct-shadow-pull (main.cpp:175)
    return T;
}
// The reference's DCT schedule (main.cpp:3800-3833, 4100-4120 on the CPU branch): level 0 is a continuous
// plane clamped to [-1,1] until iteration start_it, where the host probe fits the scale codes and the plane
// goes live (Decoder::dct_fit_all); every refit_every iterations after that, up to refit_until_it and short
// of the last iteration, the probe is re-run and the plane re-snapped from the shadow (Decoder::dct_refit).
void* ref_train_create_dct_sched(const OrModel* m, const OrTrainCfg* c, const float* z, const float* p, const float* tgt,
                                 const OrDct* d, float lambda, int rate_es, int rate_trunc, int start_it, int refit_every,
                                 int refit_until_it) {
    RefTrain* T = (RefTrain*)ref_train_create(m, c, z, p, tgt);
    Decoder& D = T->R.D;
    D.dct = dct_level_of(d);
    D.dct.live = false;
    D.dct.lambda = lambda; D.dct.rate_es = rate_es != 0; D.dct.rate_trunc = rate_trunc != 0;
    D.dct.refit_every = refit_every; D.dct.refit_until_it = refit_until_it;
    T->dct_start_it = start_it;
    T->shadow_pull = 0.01f;
    D.qes_refresh();   // the pre-start clamp of level 0 (main.cpp:3786)
    return T;
}
void ref_train_set_shadow_pull(void* h, float f) { ((RefTrain*)h)->shadow_pull = f; }
// --dct-shadow-pull on the CPU branch, as main.cpp:4142-4146 writes it, compiled under this build's flags.
void ref_shadow_pull(float* z, const float* zq, long long n, float f) {
    for (long long i = 0; i < n; i++) z[i] += f * (zq[i] - z[i]);
}
double ref_train_iter(void* h, int it, int iters) {
    RefTrain& T = *(RefTrain*)h;
    Decoder& D = T.R.D; const Options& o = T.R.o;
    double batch_loss = 0, diff_std = 0;
    const bool fd = it >= T.fd_from;
    if (it == T.fd_from) T.mt.adam.init(D.mlp.size());
    if (D.dct.on && !D.dct.live && it == T.dct_start_it) D.dct_fit_all(it);
    if (D.dct.live && D.dct.refit_every > 0 && it < iters && it != T.dct_start_it && it <= D.dct.refit_until_it &&
        it % D.dct.refit_every == 0) {
        size_t m1 = 0, m2 = 0;
        D.dct_refit(it, m1, m2);
    }
    T.mt.cur_it = it;
    batch_loss = fd ? T.mt.step_fd(D, T.R.target, T.rng, o, diff_std) : T.mt.step(D, T.R.target, T.rng, o, diff_std);
    if (!(o.qat > 0 && D.lat.lv.size() == 1)) T.lt.step(D, T.R.target, T.rng, o);
    if (D.dct.live && T.shadow_pull > 0.0f) {
        const size_t o0 = D.lat.lv[0].off, n0 = D.lat.lv[0].size();
        ref_shadow_pull(D.lat.z.data() + o0, D.zq.data() + o0, (long long)n0, T.shadow_pull);
        D.qes_refresh();
    }
    if (o.qat > 0 && (it % o.qat_every == 0 || it == iters)) qat_search(D, T.R.target, o.qat_ch);
    return batch_loss;
}
// The decode buffer (the snapped copy once a DCT or --qes level is live, otherwise the shadow).
void ref_train_get_zdec(void* h, float* zdec) {
    const Decoder& D = ((RefTrain*)h)->R.D;
    memcpy(zdec, D.zdec(), D.lat.z.size() * sizeof(float));
}
// --write-ntcb's rounding of the final weights to fp16 values (main.cpp:2472-2481, 4160); 0 if a weight has no fp16 value.
int ref_train_round_fp16(void* h) {
    size_t changed = 0; float maxdw = 0.0f;
    return ntcb_mlp_round_fp16(((RefTrain*)h)->R.D.mlp.p, changed, maxdw) ? 1 : 0;
}
// The loop's whole state in a file (latent, decode buffer, weights, both Adam states, the latent step counter,
// the DCT level's codes, symbols and flags), so that a long fixture run can be resumed. Returns 1 on success.
}   // extern "C"
namespace {
template <class T> void put_vec(FILE* f, const std::vector<T>& v) {
    const uint64_t n = v.size();
    fwrite(&n, sizeof(n), 1, f);
    if (n) fwrite(v.data(), sizeof(T), n, f);
}
template <class T> bool get_vec(FILE* f, std::vector<T>& v) {
    uint64_t n = 0;
    if (fread(&n, sizeof(n), 1, f) != 1) return false;
    v.resize(n);
    return n == 0 || fread(v.data(), sizeof(T), n, f) == n;
}
}   // namespace
extern "C" {
int ref_train_save(void* h, const char* path) {
    RefTrain& T = *(RefTrain*)h;
    Decoder& D = T.R.D;
    FILE* f = fopen(path, "wb");
    if (!f) return 0;
    const int32_t ints[8] = { T.mt.adam.t, T.lt.adam.t, T.lt.step_no, D.dct.live ? 1 : 0, D.dct.refits, D.dct.refitted_at,
                              D.dct.fitted_at, 0 };
    fwrite(ints, sizeof(ints), 1, f);
    put_vec(f, D.lat.z); put_vec(f, D.zq); put_vec(f, D.mlp.p);
    put_vec(f, T.mt.adam.m); put_vec(f, T.mt.adam.v); put_vec(f, T.lt.adam.m); put_vec(f, T.lt.adam.v);
    put_vec(f, D.dct.code); put_vec(f, D.dct.sym); put_vec(f, D.dct.bits);
    const bool ok = fflush(f) == 0;
    return (fclose(f) == 0 && ok) ? 1 : 0;
}
int ref_train_load(void* h, const char* path) {
    RefTrain& T = *(RefTrain*)h;
    Decoder& D = T.R.D;
    FILE* f = fopen(path, "rb");
    if (!f) return 0;
    int32_t ints[8];
    bool ok = fread(ints, sizeof(ints), 1, f) == 1;
    ok = ok && get_vec(f, D.lat.z) && get_vec(f, D.zq) && get_vec(f, D.mlp.p);
    ok = ok && get_vec(f, T.mt.adam.m) && get_vec(f, T.mt.adam.v) && get_vec(f, T.lt.adam.m) && get_vec(f, T.lt.adam.v);
    ok = ok && get_vec(f, D.dct.code) && get_vec(f, D.dct.sym) && get_vec(f, D.dct.bits);
    fclose(f);
    if (!ok) return 0;
    T.mt.adam.t = ints[0]; T.lt.adam.t = ints[1]; T.lt.step_no = ints[2];
    D.dct.live = ints[3] != 0; D.dct.refits = ints[4]; D.dct.refitted_at = ints[5]; D.dct.fitted_at = ints[6];
    return 1;
}
// The scale codes of the live DCT level.
void ref_train_get_dct_codes(void* h, uint8_t* code) {
    const DctLevel& Q = ((RefTrain*)h)->R.D.dct;
    memcpy(code, Q.code.data(), Q.code.size());
}
void ref_train_get(void* h, float* z, float* p) {
    RefTrain& T = *(RefTrain*)h;
    if (z) memcpy(z, T.R.D.lat.z.data(), T.R.D.lat.z.size() * sizeof(float));
    if (p) memcpy(p, T.R.D.mlp.p.data(), T.R.D.mlp.p.size() * sizeof(float));
}
void ref_train_destroy(void* h) { delete (RefTrain*)h; }
int ref_omp_threads() {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

}   // extern "C"
