// ntc_cuda::Trainer on gfx950: buffer ownership, the envelope checks, and the per-call kernel
// sequences. Every launch goes to the trainer's own stream; every method that reads or fills a
// host buffer synchronizes that stream before returning, as the reference's blocking copies do.
//
// Reference: cuda/ntc_cuda.cu:699-1181 (Trainer::Impl, init, the step drivers) for the interface
// contract; main.cpp for the arithmetic each kernel restates.
#include <math.h>
#include <string.h>

#include <algorithm>

#include "shapes.hpp"
#include "jit.hpp"
#include "trainer_impl.hpp"

using namespace ntc_hip;

namespace {

[[noreturn]] void die(const char* msg) {
    fprintf(stderr, "ntc_hip backend: %s\n", msg);
    exit(1);
}

template <class T>
void dev_alloc(T** p, size_t n) {
    *p = nullptr;
    if (n) NTC_CHECK(ntc_hip::ntc_malloc((void**)p, n * sizeof(T)));
}
template <class T>
void dev_free(T*& p) {
    if (p) { (void)ntc_hip::ntc_free(p); p = nullptr; }
}

// Pixel footprint of every texel row / column of one level: the pixels whose tap reads the
// texel (nearest: the cell, as qat_search derives it, main.cpp:2092-2094; bilinear: x0 == t or
// x1 == t with x1 != x0, the distinct-tap rule of the scatter, main.cpp:2023-2028). Both are
// contiguous ranges because the taps are monotone in the pixel coordinate.
bool footprint_ranges(int n_px, int n_tex, bool nearest, std::vector<int>& b, std::vector<int>& e) {
    b.assign(n_tex, n_px); e.assign(n_tex, 0);
    std::vector<int> cnt(n_tex, 0);
    for (int p = 0; p < n_px; p++) {
        const Tap t = tap_of(n_tex, 1, nearest, pixel_u(p, n_px), 0.5f);
        const int hit[2] = { t.x0, t.x1 };
        for (int h = 0; h < (t.x1 != t.x0 ? 2 : 1); h++) {
            const int x = hit[h];
            b[x] = std::min(b[x], p); e[x] = std::max(e[x], p + 1); cnt[x]++;
        }
    }
    for (int x = 0; x < n_tex; x++) if (cnt[x] && cnt[x] != e[x] - b[x]) return false;
    return true;
}

void snap_latent_impl(Impl& I) {
    if (!I.qes && !I.dct) return;
    launch_qes_snap(I);
    if (I.dct) {
        if (I.dct_live) launch_dct_snap(I);
        else launch_dct_clamp0(I);
    }
}

void ensure_part(Impl& I, size_t need) {
    if (need <= I.part_cap) return;
    dev_free(I.part);
    I.part_cap = need;
    dev_alloc(&I.part, need);
}

void ensure_wsets(Impl& I, size_t need) {
    if (need <= I.wsets_cap) return;
    dev_free(I.wsets);
    I.wsets_cap = need;
    dev_alloc(&I.wsets, need);
}

// A latent step's pairs run in groups of at most G pairs (its Gaussians and per-pixel differences, G x (nz + W H)
// floats, within kLatGroupBytes unless a group size is set): the memory of a step no longer grows with K. The
// DCT rate pass's bit differences (K x n, n = level 0's texels / 64) are kept for every pair.
constexpr size_t kLatGroupBytes = (size_t)1 << 30;
int lat_group_of(const Impl& I, int K) {
    int G = I.lat_group;
    if (G <= 0) G = (int)std::min<size_t>(65535, std::max<size_t>(1, kLatGroupBytes / (sizeof(float) * ((size_t)I.nz + I.npix))));
    return std::min(std::min(G, 65535), K);
}
void ensure_lat(Impl& I, int G, int K) {
    if (G > I.Kcap) {
        dev_free(I.eps_lat); dev_free(I.dpix); dev_free(I.eps_ahead);
        I.ahead_step = -1;
        I.Kcap = G;
        dev_alloc(&I.eps_lat, (size_t)G * I.nz);
        dev_alloc(&I.dpix, (size_t)G * I.npix);
    }
    if (G >= K && !I.eps_ahead) dev_alloc(&I.eps_ahead, (size_t)I.Kcap * I.nz);   // a one-group step draws the next one's Gaussians
    if (I.dct && K > I.Dcap) {
        dev_free(I.dct_dbits);
        I.Dcap = K;
        dev_alloc(&I.dct_dbits, (size_t)K * I.ddct.n);
    }
}

void sync(Impl& I) { NTC_CHECK(hipStreamSynchronize(I.stream)); }

}   // namespace

namespace ntc_hip {
std::atomic<long long> g_device_allocs{ 0 }, g_device_frees{ 0 };
// The decoder sensitivity probe on the device (the host's dct_probe_codes, main.cpp:1001-1032).
void dct_probe_impl(Impl& I, uint8_t* code, float* gain) {
    if (!I.dct) die("dct_probe without --dct-q in the model description");
    launch_dct_probe(I, I.dct_probe_code, I.dct_gain);
    if (code) NTC_CHECK(hipMemcpyAsync(code, I.dct_probe_code, (size_t)I.ddct.n, hipMemcpyDeviceToHost, I.stream));
    if (gain) NTC_CHECK(hipMemcpyAsync(gain, I.dct_gain, (size_t)I.ddct.n * sizeof(float), hipMemcpyDeviceToHost, I.stream));
    if (code || gain) sync(I);   // the host reads what was copied; without an output the launch stays enqueued
}
// Decoder::dct_refit (main.cpp:1672-1680) on the device: probe, replace the codes, re-snap (qes_refresh).
void dct_refit_impl(Impl& I, uint8_t* code) {
    if (!I.dct || !I.dct_live) die("dct_refit before set_dct");
    launch_dct_probe(I, I.dct_code, nullptr);
    snap_latent_impl(I);
    if (code) {
        NTC_CHECK(hipMemcpyAsync(code, I.dct_code, (size_t)I.ddct.n, hipMemcpyDeviceToHost, I.stream));
        sync(I);
    }
}

// The print path's error figures without a download (mse_of, main.cpp:1764-1788): decode the decode
// buffer - or, as decode_full, a latent the host passes (the post-hoc quantized one of bitrate_stats,
// main.cpp:4172-4174) - on the device, then the exact per-texture sums of squared 8-bit differences.
void decode_error_impl(Impl& I, const float* z_host, int ew, int eh, double* tex_mse, double* weighted) {
    if (I.d.nout % 3 != 0) die("decode_error needs RGB textures (nout a multiple of 3)");
    if (ew <= 0 || ew > I.d.W) ew = I.d.W;
    if (eh <= 0 || eh > I.d.H) eh = I.d.H;
    const size_t blocks = ((size_t)ew * eh + 255) / 256;
    unsigned long long* part = nullptr;
    NTC_CHECK(ntc_hip::ntc_malloc(&part, blocks * 4 * sizeof(unsigned long long)));
    const float* zsrc = I.zdec;
    if (z_host) {
        NTC_CHECK(hipMemcpyAsync(I.ztmp, z_host, I.nz * sizeof(float), hipMemcpyHostToDevice, I.stream));
        zsrc = I.ztmp;
    }
    launch_decode(I, zsrc);
    launch_u8_sse(I, ew, eh, part);
    std::vector<unsigned long long> h(blocks * 4);
    NTC_CHECK(hipMemcpyAsync(h.data(), part, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost, I.stream));
    sync(I);
    NTC_CHECK(ntc_hip::ntc_free(part));
    const int T = I.d.nout / 3;
    const double npix = (double)ew * eh;
    double ws = 0.0;
    for (int t = 0; t < T; t++) {
        unsigned long long sse = 0;
        for (size_t b = 0; b < blocks; b++) sse += h[b * 4 + t];
        if (tex_mse) tex_mse[t] = (double)sse / (3.0 * npix);
        ws += (double)I.d.cw[3 * t] * (double)sse;
    }
    if (weighted) *weighted = ws / (3.0 * (double)I.d.wsum * npix);
}

// The decoder's product (ntc_decode.cpp's RGB8 output, save_png's rounding) without the float image
// crossing PCIe: decode on the device, round to 8 bits there, download W x H x nout bytes.
void decode_rgb8_impl(Impl& I, uint8_t* out) {
    const size_t n = (size_t)I.npix * I.d.nout;
    uint8_t* d = nullptr;
    NTC_CHECK(ntc_hip::ntc_malloc(&d, n));
    launch_decode(I, I.zdec);
    launch_pack_u8(I, d);
    NTC_CHECK(hipMemcpyAsync(out, d, n, hipMemcpyDeviceToHost, I.stream));
    sync(I);
    NTC_CHECK(ntc_hip::ntc_free(d));
}

void resolve_times(Impl& I) {
    bool any = false;
    for (auto& kv : I.times) if (!kv.second.pending.empty()) any = true;
    if (!any) return;
    NTC_CHECK(hipStreamSynchronize(I.stream));
    for (auto& kv : I.times) {
        for (auto& ev : kv.second.pending) {
            float ms = 0.0f;
            NTC_CHECK(hipEventElapsedTime(&ms, ev.first, ev.second));
            kv.second.total_ms += ms;
            kv.second.launches++;
            (void)hipEventDestroy(ev.first); (void)hipEventDestroy(ev.second);
        }
        kv.second.pending.clear();
    }
}
}   // namespace ntc_hip

namespace ntc_cuda {

Trainer::Trainer() : im(new Impl) {}

Trainer::~Trainer() {
    Impl& I = *im;
    if (I.stream) {   // never initialised: nothing on the device to release
        (void)hipStreamSynchronize(I.stream);
        for (auto& kv : I.times)
            for (auto& ev : kv.second.pending) { (void)hipEventDestroy(ev.first); (void)hipEventDestroy(ev.second); }
        dev_free(I.z); dev_free(I.zq); dev_free(I.zgrad); dev_free(I.zm); dev_free(I.zv); dev_free(I.ztmp);
        dev_free(I.w); dev_free(I.wgrad); dev_free(I.wm); dev_free(I.wv);
        dev_free(I.tgt); dev_free(I.img); dev_free(I.feat); dev_free(I.btgt); dev_free(I.bidx); dev_free(I.lay1);
        dev_free(I.wsets); dev_free(I.eps_mlp); dev_free(I.gpart); dev_free(I.part); dev_free(I.dl); dev_free(I.lsum); dev_free(I.hh);
        dev_free(I.eps_lat); dev_free(I.eps_ahead); dev_free(I.dpix); dev_free(I.ranges); dev_free(I.qat_grid); dev_free(I.qat_bits);
        dev_free(I.qes_dev); dev_free(I.qgrid);
        dev_free(I.zpost); dev_free(I.st_part); dev_free(I.st_keys); dev_free(I.st_hist); dev_free(I.st_dct); dev_free(I.st_sse);
        dev_free(I.dct_sym); dev_free(I.dct_code); dev_free(I.dct_step); dev_free(I.dct_bits); dev_free(I.dct_dbits); dev_free(I.dct_tn); dev_free(I.dct_probe_code); dev_free(I.dct_gain);
        (void)hipStreamDestroy(I.stream);
    }
    delete im;
}

bool Trainer::init(const ModelDesc& d, const float* z, const float* p, const float* target, std::string& why) {
    Impl& I = *im;
    if (I.stream) { why = "the trainer is already initialised"; return false; }
    I.d = d;
    // ---- envelope (the reference's, cuda/ntc_cuda.cu:755-785, without its 48 KiB shared-memory limit)
    if (d.nlev < 1 || d.nlev > MAX_LEVELS) { why = "bad level count"; return false; }
    if (d.nhidden < 0 || d.nhidden > MAX_HIDDEN) { why = "too many hidden layers"; return false; }
    if (d.npos < 0 || d.npos > MAX_POS) { why = "too many positional features"; return false; }
    int need = d.nin;
    for (int l = 0; l < d.nhidden; l++) need = std::max(need, d.hidden[l]);
    if (need > kMaxWidth) { why = "at most 64 units per layer (input and hidden)"; return false; }
    if (d.nout < 1 || d.nout > MAX_OUT) { why = "too many MLP outputs"; return false; }
    if (d.lv[0].C > MAX_CH) { why = "at most 16 level-0 channels"; return false; }
    {
        int nin = 2 * d.npos;
        for (int l = 0; l < d.nlev; l++) {
            if (d.lv[l].W < 1 || d.lv[l].H < 1 || d.lv[l].C < 1) { why = "empty latent level"; return false; }
            nin += d.lv[l].C;
        }
        if (nin != d.nin) { why = "nin differs from the latent channels plus the positional features"; return false; }
        for (int q = 0; q < d.npos; q++) {
            if (d.pos[q].kind != PK_UV && d.pos[q].kind != PK_LV1LOCAL) { why = "unknown positional feature kind"; return false; }
            if (d.pos[q].kind == PK_LV1LOCAL && d.nlev < 2) { why = "lv1local needs a second latent level"; return false; }
        }
        size_t off = 0;
        for (int l = 0; l < d.nlev; l++) {
            if (d.lv[l].off != off) { why = "latent levels must be concatenated in order"; return false; }
            off += (size_t)d.lv[l].W * d.lv[l].H * d.lv[l].C;
        }
        if (off >= ((size_t)1 << 30)) { why = "latents of at most 2^30 values (32-bit element offsets)"; return false; }
    }
    for (int l = 0; l < d.nhidden; l++) if (d.hidden[l] < 1) { why = "empty hidden layer"; return false; }
    I.qes = false;
    for (int l = 0; l < d.nlev; l++)
        if (d.qes_bits[l] > 0) {
            I.qes = true;
            if (d.qes_bits[l] < 2 || d.qes_bits[l] > 12) { why = "--qes bits out of range"; return false; }
            if (d.lv[l].C > MAX_QES_CH) { why = "at most 64 channels on a --qes level"; return false; }
        }
    if (d.qat > 0) {
        if (!d.qat_grid) { why = "--qat needs the host grid table"; return false; }
        if (!d.lv[0].nearest) { why = "--qat needs nearest sampling on level 0"; return false; }
        for (int c = 0; c < d.lv[0].C; c++)
            if (d.qat_bits[c] < 1 || d.qat_bits[c] > 8) { why = "--qat bits out of range"; return false; }
    }
    I.dct = d.dct != 0;
    I.dct_live = false;
    if (I.dct) {
        if (d.dct_N != 8) { why = "--dct-q: block size 8 only"; return false; }
        if (d.dct_C < 1 || d.dct_C > MAX_DCT_CH || d.dct_C != d.lv[0].C) { why = "--dct-q: level 0 must have 1..4 channels (= dct_C)"; return false; }
        if (!d.lv[0].nearest || d.lv[0].W != d.W || d.lv[0].H != d.H || d.W % 8 != 0 || d.H % 8 != 0) {
            why = "--dct-q: level 0 must be a full-resolution nearest level with a size that is a multiple of 8"; return false;
        }
        if (!d.dct_basis) { why = "--dct-q needs the host basis table"; return false; }
        if (!d.dct_zigzag) { why = "--dct-q needs the host zigzag table"; return false; }
        if (d.dct_dc_step < 1 || d.dct_dc_step > 64) { why = "--dct-q: DC step out of range"; return false; }
    }
    if (d.W < 1 || d.H < 1 || (size_t)d.W * d.H >= ((size_t)1 << 28)) { why = "images below 2^28 pixels only"; return false; }
    if (d.max_pairs < 1 || d.max_batch < 1) { why = "bad pair / batch counts"; return false; }
    {
        int in = d.nin; long long n = 0;
        for (int l = 0; l < d.nhidden; l++) { n += (long long)d.hidden[l] * in + d.hidden[l]; in = d.hidden[l]; }
        n += (long long)d.nout * in + d.nout;
        I.P = (int)n;
    }

    // ---- device
    if (hipGetDevice(&I.device) != hipSuccess) { why = "no HIP device"; return false; }
    hipDeviceProp_t prop;
    NTC_CHECK(hipGetDeviceProperties(&prop, I.device));
    I.dev_name = prop.name; I.arch = prop.gcnArchName; I.cus = prop.multiProcessorCount;
    NTC_CHECK(hipRuntimeGetVersion(&I.rt_ver));
    if (!noise_fix_for_device(I.device, I.noise, why)) return false;
    if (!noalloc_scratch_setup(I.device, why)) return false;
    NTC_CHECK(hipStreamCreateWithFlags(&I.stream, hipStreamNonBlocking));

    // ---- model description
    I.npix = (size_t)d.W * d.H;
    I.nz = 0;
    for (int l = 0; l < d.nlev; l++) I.nz += (size_t)d.lv[l].W * d.lv[l].H * d.lv[l].C;
    DevModel& m = I.dm;
    memset(&m, 0, sizeof(m));
    m.W = d.W; m.H = d.H; m.npix = (int)I.npix; m.nout = d.nout; m.nin = d.nin; m.nlev = d.nlev; m.npos = d.npos; m.nl = d.nhidden;
    std::vector<int> ranges;
    for (int l = 0; l < d.nlev; l++) {
        DevLevel& L = m.lv[l];
        L.W = d.lv[l].W; L.H = d.lv[l].H; L.C = d.lv[l].C; L.nearest = d.lv[l].nearest ? 1 : 0; L.off = (long long)d.lv[l].off;
        L.rng = (int)ranges.size();
        std::vector<int> xb, xe, yb, ye;
        if (!footprint_ranges(d.W, L.W, L.nearest != 0, xb, xe) || !footprint_ranges(d.H, L.H, L.nearest != 0, yb, ye)) {
            why = "internal: a texel footprint is not contiguous"; return false;
        }
        ranges.insert(ranges.end(), xb.begin(), xb.end()); ranges.insert(ranges.end(), xe.begin(), xe.end());
        ranges.insert(ranges.end(), yb.begin(), yb.end()); ranges.insert(ranges.end(), ye.begin(), ye.end());
        if (l == 0) {   // level 0 with one pixel per texel (texel x covers exactly pixel x): the selector search's per-pixel form
            bool unit = L.nearest && L.W == d.W && L.H == d.H;
            for (int x = 0; unit && x < L.W; x++) unit = xb[x] == x && xe[x] == x + 1;
            for (int y = 0; unit && y < L.H; y++) unit = yb[y] == y && ye[y] == y + 1;
            I.lv0_unit_cells = unit;
        }
    }
    for (int q = 0; q < d.npos; q++) m.pos[q] = d.pos[q].kind;
    for (int l = 0; l < d.nhidden; l++) m.hidden[l] = d.hidden[l];
    m.leak = d.leak; m.clamp_out = d.clamp_out ? 1 : 0;
    m.fold_c = (1.0f - d.leak) / (1.0f + d.leak);
    for (int c = 0; c < MAX_OUT; c++) m.cw[c] = c < d.nout ? d.cw[c] : 0.0f;
    m.wsum = d.wsum;
    m.inv_px = 1.0f / (3.0f * d.wsum * (float)d.W * (float)d.H);
    m.P = I.P;
    m.nz = (long long)I.nz;
    I.shape_name = dispatch_shape(m, [](auto) {});
    I.jit = nullptr;

    // ---- buffers
    dev_alloc(&I.ranges, ranges.size());
    NTC_CHECK(hipMemcpy(I.ranges, ranges.data(), ranges.size() * sizeof(int), hipMemcpyHostToDevice));
    dev_alloc(&I.z, I.nz); dev_alloc(&I.zgrad, I.nz); dev_alloc(&I.zm, I.nz); dev_alloc(&I.zv, I.nz); dev_alloc(&I.ztmp, I.nz);
    if (I.qes || I.dct) {
        dev_alloc(&I.zq, I.nz);
        dev_alloc(&I.qes_dev, 1);
        QesDesc q0; memset(&q0, 0, sizeof(q0));
        for (int l = 0; l < d.nlev; l++) q0.bits[l] = d.qes_bits[l];
        NTC_CHECK(hipMemcpy(I.qes_dev, &q0, sizeof(q0), hipMemcpyHostToDevice));
        I.qes_h = q0;
        if (I.qes) dev_alloc(&I.qgrid, (size_t)MAX_LEVELS * MAX_QES_CH * 4096);
        I.zdec = I.zq;
    } else {
        I.zdec = I.z;
    }
    if (I.dct) {
        DevDct& D = I.ddct;
        memset(&D, 0, sizeof(D));
        D.C = d.dct_C; D.BW = d.W / 8; D.BH = d.H / 8; D.dc_step = d.dct_dc_step; D.deadzone = 1; D.lo_w16 = 16;
        D.n = D.BW * D.BH * D.C;
        memcpy(D.basis, d.dct_basis, sizeof(D.basis));
        memcpy(D.zigzag, d.dct_zigzag, sizeof(D.zigzag));
        dev_alloc(&I.dct_sym, (size_t)D.n * 64); dev_alloc(&I.dct_code, (size_t)D.n); dev_alloc(&I.dct_step, (size_t)D.C * 16 * 64);
        dev_alloc(&I.dct_bits, (size_t)D.n); dev_alloc(&I.dct_tn, 2 * (size_t)D.n);
        dev_alloc(&I.dct_probe_code, (size_t)D.n); dev_alloc(&I.dct_gain, (size_t)D.n);
        NTC_CHECK(hipMemset(I.dct_sym, 0, (size_t)D.n * 64 * sizeof(int16_t)));
        NTC_CHECK(hipMemset(I.dct_code, 0, (size_t)D.n));
        NTC_CHECK(hipMemset(I.dct_step, 0, (size_t)D.C * 16 * 64 * sizeof(int)));
        NTC_CHECK(hipMemset(I.dct_bits, 0, (size_t)D.n * sizeof(int32_t)));
        NTC_CHECK(hipMemset(I.dct_tn, 0, 2 * (size_t)D.n * sizeof(int)));
    }
    dev_alloc(&I.w, I.P); dev_alloc(&I.wgrad, I.P); dev_alloc(&I.wm, I.P); dev_alloc(&I.wv, I.P);
    dev_alloc(&I.tgt, I.npix * d.nout); dev_alloc(&I.img, I.npix * d.nout);
    I.Mcap = d.max_batch;
    // the matrix-core population evaluation reads whole 16-slot tiles and 4-input k-steps: zero feature rows
    // up to minibatch_rows(nin) and kMinibatchSlack floats past the last row of each array
    const size_t nfeat = (size_t)I.Mcap * minibatch_rows(d.nin) + kMinibatchSlack;
    dev_alloc(&I.feat, nfeat); dev_alloc(&I.btgt, (size_t)I.Mcap * d.nout + kMinibatchSlack); dev_alloc(&I.bidx, (size_t)I.Mcap);
    NTC_CHECK(hipMemset(I.feat, 0, nfeat * sizeof(float)));
    NTC_CHECK(hipMemset(I.btgt, 0, ((size_t)I.Mcap * d.nout + kMinibatchSlack) * sizeof(float)));
    I.pairs_cap = d.max_pairs;
    dev_alloc(&I.eps_mlp, (size_t)I.pairs_cap * I.P);
    I.gpart_cap = (size_t)((I.pairs_cap + 127) / 128) * I.P;
    dev_alloc(&I.gpart, I.gpart_cap);
    if (!pop_on_matrix_cores(I)) ensure_wsets(I, (size_t)2 * I.pairs_cap * I.P);   // the matrix-core ES step needs none
    ensure_part(I, (size_t)2 * (std::max(I.pairs_cap, I.P + 1) * 4 + 2048));
    dev_alloc(&I.dl, (size_t)std::max(I.pairs_cap, I.P)); dev_alloc(&I.lsum, (size_t)I.pairs_cap); dev_alloc(&I.hh, (size_t)I.P);
    if (d.qat > 0) {
        dev_alloc(&I.qat_grid, 9 * 257); dev_alloc(&I.qat_bits, MAX_CH);
        NTC_CHECK(hipMemcpy(I.qat_grid, d.qat_grid, sizeof(float) * 9 * 257, hipMemcpyHostToDevice));
        NTC_CHECK(hipMemcpy(I.qat_bits, d.qat_bits, sizeof(int) * MAX_CH, hipMemcpyHostToDevice));
    }
    NTC_CHECK(hipMemset(I.zm, 0, I.nz * sizeof(float))); NTC_CHECK(hipMemset(I.zv, 0, I.nz * sizeof(float)));
    NTC_CHECK(hipMemset(I.wm, 0, I.P * sizeof(float))); NTC_CHECK(hipMemset(I.wv, 0, I.P * sizeof(float)));
    NTC_CHECK(hipMemcpy(I.tgt, target, I.npix * d.nout * sizeof(float), hipMemcpyHostToDevice));
    if (I.shape_name == "runtime") {   // a shape shapes.hpp does not list: the fixed-shape kernels compiled for it now
        std::string jwhy;
        JitShape js{};
        if (jit_prepare(I, jwhy) && jit_shape_of(I.dm, js)) {
            char b[64];
            snprintf(b, sizeof(b), "%d+%d+%d|%dpos|", js.C0, js.C1, js.C2, js.npos);
            std::string n = b;
            if (js.uniform()) n += std::to_string(js.H[0]) + "x" + std::to_string(js.NL);
            else for (int l = 0; l < js.NL; l++) n += (l ? "," : "") + std::to_string(js.H[l]);
            I.shape_name = n + "|" + std::to_string(js.nout) + " (specialised at init)";
        } else {
            fprintf(stderr, "ntc_hip backend: the runtime-shaped kernels run this model (%s)\n", jwhy.c_str());
        }
    }
    I.pop_pair = pop_pair_possible(I);
    if (I.pop_pair) {
        const size_t n = (size_t)I.d.hidden[0] * I.Mcap + kMinibatchSlack;
        dev_alloc(&I.lay1, n);
        NTC_CHECK(hipMemset(I.lay1, 0, n * sizeof(float)));
    }
    upload_model(z, p);
    return true;
}

std::string Trainer::banner() const {
    const Impl& I = *im;
    char buf[320];
    snprintf(buf, sizeof(buf), "%s (%s, %d CUs), HIP runtime %d.%d, MLP shape %s", I.dev_name.c_str(), I.arch.c_str(), I.cus,
             I.rt_ver / 10000000, (I.rt_ver / 100000) % 100, I.shape_name.c_str());
    return buf;
}

void Trainer::upload_model(const float* z, const float* p) {
    Impl& I = *im;
    NTC_CHECK(hipMemcpyAsync(I.z, z, I.nz * sizeof(float), hipMemcpyHostToDevice, I.stream));
    NTC_CHECK(hipMemcpyAsync(I.w, p, I.P * sizeof(float), hipMemcpyHostToDevice, I.stream));
    snap_latent_impl(I);
    sync(I);
}

void Trainer::download_model(float* z, float* p) {
    Impl& I = *im;
    NTC_CHECK(hipMemcpyAsync(z, I.z, I.nz * sizeof(float), hipMemcpyDeviceToHost, I.stream));
    NTC_CHECK(hipMemcpyAsync(p, I.w, I.P * sizeof(float), hipMemcpyDeviceToHost, I.stream));
    sync(I);
}

void Trainer::set_qes(const QesDesc& q, const float* grid, size_t grid_n) {
    Impl& I = *im;
    if (!I.qes) die("set_qes without a --qes level in the model description");
    if (grid_n > (size_t)MAX_LEVELS * MAX_QES_CH * 4096) die("--qes grid table too large");
    I.qes_h = q;
    NTC_CHECK(hipMemcpyAsync(I.qes_dev, &q, sizeof(q), hipMemcpyHostToDevice, I.stream));
    if (grid_n) NTC_CHECK(hipMemcpyAsync(I.qgrid, grid, grid_n * sizeof(float), hipMemcpyHostToDevice, I.stream));
    snap_latent_impl(I);
    sync(I);
}

// Reads and writes device memory only: enqueued on the trainer's stream, as the reference's kernels are
// (cuda/ntc_cuda.cu:978-988); the next call that copies to or from the host waits for it.
void Trainer::snap_latent() { snap_latent_impl(*im); }

void Trainer::shadow_pull(size_t off, size_t n, float f) {
    Impl& I = *im;
    if (!I.zq || n == 0) return;
    if (off + n > I.nz) die("shadow_pull range outside the latent");
    const size_t n0 = (size_t)I.d.lv[0].W * I.d.lv[0].H * I.d.lv[0].C;
    if (I.dct && I.dct_live && off == (size_t)I.dm.lv[0].off && n == n0 && f != 0.0f) {
        // the live plane as a whole: the pull inside the re-snap's launch (the other levels' shadow did not move, so
        // their snapped values stand)
        launch_dct_snap(I, f);
        return;
    }
    launch_shadow_pull(I, off, n, f);
    snap_latent_impl(I);
}

void Trainer::download_zq(float* zq) {
    Impl& I = *im;
    NTC_CHECK(hipMemcpyAsync(zq, I.zdec, I.nz * sizeof(float), hipMemcpyDeviceToHost, I.stream));
    sync(I);
}

void Trainer::set_dct(const DctDesc& dd, const uint8_t* code, const int16_t* sym, const int* step) {
    Impl& I = *im;
    if (!I.dct) die("set_dct without --dct-q in the model description");
    if (dd.C != I.d.dct_C || dd.BW * dd.BH * dd.C != I.ddct.n || dd.N != 8) die("set_dct description mismatch");
    DevDct& D = I.ddct;
    D.live = 1; D.dc_step = dd.dc_step; D.deadzone = dd.deadzone; D.lo_w16 = dd.lo_w16;
    D.rate_es = dd.rate_es; D.rate_trunc = dd.rate_trunc; D.rate_scale = dd.rate_scale;
    for (int k = 0; k < 16; k++) D.lam_t16[k] = dd.lam_t16[k];
    NTC_CHECK(hipMemcpyAsync(I.dct_step, step, sizeof(int) * 16 * 64 * dd.C, hipMemcpyHostToDevice, I.stream));
    NTC_CHECK(hipMemcpyAsync(I.dct_code, code, (size_t)D.n, hipMemcpyHostToDevice, I.stream));
    NTC_CHECK(hipMemcpyAsync(I.dct_sym, sym, (size_t)D.n * 64 * sizeof(int16_t), hipMemcpyHostToDevice, I.stream));
    I.dct_live = true;
    I.dct_rate_es = dd.rate_es != 0; I.dct_rate_trunc = dd.rate_trunc != 0;
    launch_dct_recon(I);
    sync(I);
}

void Trainer::download_dct(int16_t* sym, uint8_t* code) {
    Impl& I = *im;
    if (!I.dct) return;
    NTC_CHECK(hipMemcpyAsync(sym, I.dct_sym, (size_t)I.ddct.n * 64 * sizeof(int16_t), hipMemcpyDeviceToHost, I.stream));
    NTC_CHECK(hipMemcpyAsync(code, I.dct_code, (size_t)I.ddct.n, hipMemcpyDeviceToHost, I.stream));
    sync(I);
}

void Trainer::download_dct_rate(int32_t* bits, int32_t* dbits_last_pair, int* ntrunc, int* nz_before, int* hits, int* evals) {
    Impl& I = *im;
    if (!I.dct) return;
    if (bits) NTC_CHECK(hipMemcpyAsync(bits, I.dct_bits, (size_t)I.ddct.n * sizeof(int32_t), hipMemcpyDeviceToHost, I.stream));
    if (dbits_last_pair) {
        if (I.dct_dbits && I.dct_last_K > 0)
            NTC_CHECK(hipMemcpyAsync(dbits_last_pair, I.dct_dbits + (size_t)(I.dct_last_K - 1) * I.ddct.n,
                                     (size_t)I.ddct.n * sizeof(int32_t), hipMemcpyDeviceToHost, I.stream));
        else memset(dbits_last_pair, 0, (size_t)I.ddct.n * sizeof(int32_t));
    }
    // the counts: sums of the last snap's per-block counts, and the pairs of the last rate pass whose
    // bits differ between the two members (the nonzero dbits)
    const size_t n = (size_t)I.ddct.n, nd = (I.dct_dbits && I.dct_last_K > 0) ? (size_t)I.dct_last_K * n : 0;
    std::vector<int> tn(2 * n), db(nd);
    NTC_CHECK(hipMemcpyAsync(tn.data(), I.dct_tn, 2 * n * sizeof(int), hipMemcpyDeviceToHost, I.stream));
    if (nd) NTC_CHECK(hipMemcpyAsync(db.data(), I.dct_dbits, nd * sizeof(int), hipMemcpyDeviceToHost, I.stream));
    sync(I);
    long long nt = 0, nzb = 0, h = 0;
    for (size_t i = 0; i < n; i++) { nt += tn[i]; nzb += tn[n + i]; }
    for (size_t i = 0; i < nd; i++) h += db[i] != 0;
    if (ntrunc) *ntrunc = (int)nt;
    if (nz_before) *nz_before = (int)nzb;
    if (hits) *hits = (int)h;
    if (evals) *evals = I.dct_evals;
}

void Trainer::mlp_step(int it, float sigma, float lr, int N, int M) {
    Impl& I = *im;
    if (N > I.pairs_cap || M > I.Mcap || N < 1 || M < 1) {
        fprintf(stderr, "ntc_hip backend: MLP step with %d pairs / %d pixels outside the buffers sized at init (%d / %d)\n", N, M,
                I.pairs_cap, I.Mcap);
        exit(1);
    }
    const int chunk = pop_chunk(I, N, M), chunks = (M + chunk - 1) / chunk;
    const bool mfma = pop_on_matrix_cores(I);
    // with the Gaussians the population kernel reads, and the first layer the pair-sharing kernel reads
    launch_batch(I, it, M, mfma && pop_reads_eps(chunks) ? N : 0, pop_pair_step(I, chunk));
    ensure_part(I, (size_t)2 * N * chunks);
    if (mfma) {
        launch_pop_eval_es(I, it, sigma, N, M, chunk, chunks);   // stages the perturbed weights itself
    } else {
        ensure_wsets(I, (size_t)2 * N * I.P);
        launch_perturb(I, it, sigma, N);
        launch_pop_eval(I, N, M, chunk, chunks);
    }
    launch_es_update(I, chunks, 3.0 * (double)I.d.wsum * (double)M, sigma, N, lr, ++I.mlp_t);
    I.last_N = N; I.last_fd = false; I.last_M = M; I.last_chunk = chunk;
}

void Trainer::mlp_step_fd(int it, float h, float lr, int M) {
    Impl& I = *im;
    if (M > I.Mcap || M < 1) {
        fprintf(stderr, "ntc_hip backend: FD step with %d pixels outside the buffers sized at init (%d)\n", M, I.Mcap);
        exit(1);
    }
    launch_batch(I, it, M);
    ensure_wsets(I, (size_t)2 * (I.P + 1) * I.P);
    launch_fd_sets(I, h);
    const int chunk = pop_chunk(I, I.P + 1, M), chunks = (M + chunk - 1) / chunk;
    ensure_part(I, (size_t)2 * (I.P + 1) * chunks);
    launch_pop_eval(I, I.P + 1, M, chunk, chunks);
    launch_fd_finish(I, chunks, 3.0 * (double)I.d.wsum * (double)M);
    launch_adam(I, I.w, I.wgrad, I.wm, I.wv, I.P, lr, ++I.mlp_t);
    I.last_N = I.P; I.last_fd = true; I.last_M = M; I.last_chunk = chunk;
}

void Trainer::reset_mlp_adam() {
    Impl& I = *im;
    launch_fill(I, I.wm, I.P, 0.0f);
    launch_fill(I, I.wv, I.P, 0.0f);
    I.mlp_t = 0;
}

void Trainer::mlp_stats(double& batch_loss, double& diff_std) {
    Impl& I = *im;
    if (I.last_N == 0) { batch_loss = 0; diff_std = 0; return; }
    if (!I.last_fd) {
        std::vector<double> dl(I.last_N), lsum(I.last_N);
        NTC_CHECK(hipMemcpyAsync(dl.data(), I.dl, I.last_N * sizeof(double), hipMemcpyDeviceToHost, I.stream));
        NTC_CHECK(hipMemcpyAsync(lsum.data(), I.lsum, I.last_N * sizeof(double), hipMemcpyDeviceToHost, I.stream));
        sync(I);
        double mean = 0, mean2 = 0, lmean = 0;
        for (int i = 0; i < I.last_N; i++) { mean += dl[i]; mean2 += dl[i] * dl[i]; lmean += lsum[i]; }
        mean /= I.last_N; mean2 /= I.last_N; lmean /= I.last_N;
        diff_std = sqrt(std::max(0.0, mean2 - mean * mean));
        batch_loss = lmean;
    } else {
        std::vector<double> dl(I.P);
        double l0 = 0;
        NTC_CHECK(hipMemcpyAsync(dl.data(), I.dl, I.P * sizeof(double), hipMemcpyDeviceToHost, I.stream));
        NTC_CHECK(hipMemcpyAsync(&l0, I.lsum, sizeof(double), hipMemcpyDeviceToHost, I.stream));
        sync(I);
        double ss = 0;
        for (int j = 0; j < I.P; j++) ss += dl[j] * dl[j];
        diff_std = sqrt(ss / I.P);
        batch_loss = l0;
    }
}

void Trainer::lat_step(int /*it*/, float sigma, float lr, int K) {
    Impl& I = *im;
    if (K < 1) die("lat_step takes at least one pair");
    const bool qat = I.d.qat > 0;
    unsigned mask = 0;
    for (int l = 0; l < I.d.nlev; l++) if (!(qat && l == 0)) mask |= 1u << l;
    const int G = lat_group_of(I, K);
    ensure_lat(I, G, K);
    const bool rate = I.dct_live && I.dct_rate_es;
    I.dct_evals = rate ? I.ddct.n * K : 0;
    if (!mask) launch_fill(I, I.zgrad, I.nz, 0.0f);
    bool direct_zq = false;
    if (mask) {
        const float scale = 1.0f / (2.0f * (float)K * sigma);
        ++I.lat_t;
        // The pairs in groups, in order: each group's gathers add its pairs to every texel's gradient after the
        // previous groups' (the reference's pair order, main.cpp:1990-2037: the same sums, bit for bit), and the
        // shadow and decode buffer stay as they are until the last group. Adam on the perturbed levels inside the
        // last group's gathers. The other levels' gradients are zero at every step of this trainer (the mask is
        // fixed by --qat at init), so their Adam moments stay zero and the reference's step leaves them exactly
        // as they are: it is skipped.
        //
        // A step that runs as one group has the next step's Gaussians drawn by its last gather launch (for step
        // lat_step_no + 1 and the same K): the next step then swaps them in and launches no draw of its own. The
        // first group's gathers start the gradient from zero, so the cleared zgrad of k_lat_eps is not needed then
        // (the levels outside the mask keep the zeros of the first step's draw: nothing writes them).
        const bool ahead = I.ahead_step == I.lat_step_no && I.ahead_K == K && G >= K && I.eps_ahead;
        if (ahead) std::swap(I.eps_lat, I.eps_ahead);
        // a DCT model without --qes whose step moves every level past the plane: the gathers' Adam steps write those
        // levels' decode copy themselves, and the snap after the step is the plane's alone
        direct_zq = I.dct && !I.qes && (mask | 1u) == (1u << I.d.nlev) - 1;
        for (int k0 = 0; k0 < K; k0 += G) {
            const int g = std::min(G, K - k0);
            const bool last = k0 + g == K;
            if (!(ahead && k0 == 0)) launch_lat_eps(I, k0, g, mask);   // the first group also clears zgrad
            launch_lat_pair(I, g, sigma, mask);
            I.lat_last_K = g;
            if (rate) launch_dct_rate_pairs(I, k0, g, sigma);
            launch_lat_gather(I, mask, k0, g, scale, rate, lr, last ? I.lat_t : 0, G >= K ? K : 0, direct_zq ? I.zq : nullptr);
        }
        I.ahead_step = G >= K ? I.lat_step_no + 1 : -1;
        I.ahead_K = K;
        if (rate) I.dct_last_K = K;
    } else {
        launch_adam(I, I.z, I.zgrad, I.zm, I.zv, I.nz, lr, ++I.lat_t);
    }
    if (direct_zq) {
        if (I.dct_live) launch_dct_snap(I);
        else launch_dct_clamp0(I);
    } else {
        snap_latent_impl(I);
    }
    I.lat_step_no++;
}

void Trainer::qat_search() {
    Impl& I = *im;
    if (I.d.qat <= 0) die("qat_search without --qat in the model description");
    launch_qat_search(I);
    if (I.zdec != I.z) {
        const size_t n0 = (size_t)I.d.lv[0].W * I.d.lv[0].H * I.d.lv[0].C;
        NTC_CHECK(hipMemcpyAsync(I.z + I.d.lv[0].off, I.zdec + I.d.lv[0].off, n0 * sizeof(float), hipMemcpyDeviceToDevice, I.stream));
    }
}

void Trainer::decode_full(const float* z_host, float* img) {
    Impl& I = *im;
    const float* zsrc = I.zdec;
    if (z_host) {
        NTC_CHECK(hipMemcpyAsync(I.ztmp, z_host, I.nz * sizeof(float), hipMemcpyHostToDevice, I.stream));
        zsrc = I.ztmp;
    }
    launch_decode(I, zsrc);
    NTC_CHECK(hipMemcpyAsync(img, I.img, I.npix * I.d.nout * sizeof(float), hipMemcpyDeviceToHost, I.stream));
    sync(I);
}

void Trainer::dct_probe(uint8_t* code, float* gain) { ntc_hip::dct_probe_impl(*im, code, gain); }
void Trainer::dct_refit(uint8_t* code) { ntc_hip::dct_refit_impl(*im, code); }
void Trainer::decode_error(const float* z_host, int ew, int eh, double* tex_mse, double* weighted) {
    ntc_hip::decode_error_impl(*im, z_host, ew, eh, tex_mse, weighted);
}
void Trainer::decode_rgb8(uint8_t* out) { ntc_hip::decode_rgb8_impl(*im, out); }
void Trainer::print_stats(int qbits, int ew, int eh, ::ntc_print_stats* out) {
    ntc_hip::print_stats_impl(*im, qbits, ew, eh, out);
}

void Trainer::debug_last_batch(std::vector<int>& bidx) const {
    Impl& I = *im;
    bidx.resize(I.last_M);
    if (I.last_M) NTC_CHECK(hipMemcpyAsync(bidx.data(), I.bidx, I.last_M * sizeof(int), hipMemcpyDeviceToHost, I.stream));
    sync(I);
}
void Trainer::debug_last_dl(std::vector<double>& dl) const {
    Impl& I = *im;
    dl.resize(I.last_N);
    if (I.last_N) NTC_CHECK(hipMemcpyAsync(dl.data(), I.dl, I.last_N * sizeof(double), hipMemcpyDeviceToHost, I.stream));
    sync(I);
}
void Trainer::debug_last_zgrad(std::vector<float>& g) const {
    Impl& I = *im;
    g.resize(I.nz);
    NTC_CHECK(hipMemcpyAsync(g.data(), I.zgrad, I.nz * sizeof(float), hipMemcpyDeviceToHost, I.stream));
    sync(I);
}

}   // namespace ntc_cuda
