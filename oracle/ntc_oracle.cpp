// CPU oracle for the ES training backend of neural_block_textures.
//
// TEST INFRASTRUCTURE ONLY: the checker the HIP kernels are compared against. The product
// library never links, loads or calls it.
//
// Every function restates a function of the reference's CPU path (main.cpp, cuda/ntc_noise.h)
// and names the lines it follows. Floating-point evaluation order: the reference's host build
// leaves FMA contraction on (GCC's default for GNU C++, with FMA hardware), and the places where
// GCC contracts a multiply into the following add are written here as explicit fmaf() calls;
// this file itself is compiled with -ffp-contract=off, so nothing else is fused. The functions the
// reference wraps in STRICT_FP_BEGIN/END (the --qes index and grid, the DCT transform,
// quantizer and rate model) contain no fmaf at all.
//
// Parity pins (tests/test_oracle_*.py): the golden vectors under tests/golden/ were written by
// the reference itself (oracle/ref_wrap.cpp includes main.cpp unmodified); the --dct-selftest
// known answers (main.cpp:1374-1540); the fp16 self-check (main.cpp:2456-2470); closed forms and
// brute force on tiny inputs.
#include "ntc_oracle.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

// ------------------------------------------------------------------ noise (cuda/ntc_noise.h)
// splitmix64's output function; the stream key and the Box-Muller draw are ntc_noise.h:20-47.
inline uint64_t mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
inline uint64_t noise_key(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index) {
    const uint64_t head = mix64(seed ^ ((uint64_t)stream << 56) ^ ((uint64_t)step << 32) ^ (uint64_t)pair);
    return mix64(head + index * 0x9E3779B97F4A7C15ull);
}
inline float radius_of(uint32_t k1) {   // sqrtf(-2 logf(u1)), u1 = (k1 + 1) / 2^24 in (0, 1]
    const float u1 = (float)(k1 + 1u) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1));
}
inline float cosine_of(uint32_t k2) {   // cosf(2 pi u2), u2 = k2 / 2^24 in [0, 1)
    const float u2 = (float)k2 * (1.0f / 16777216.0f);
    return cosf(6.283185307179586f * u2);
}
inline float gauss(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index) {
    const uint64_t h = noise_key(seed, stream, step, pair, index);
    return radius_of((uint32_t)(h >> 40)) * cosine_of((uint32_t)(h & 0xFFFFFFull));
}
enum { NS_LAT = 1, NS_MLP = 2, NS_BATCH_PIX = 3, NS_BATCH_TEX = 4 };

// ------------------------------------------------------------------ geometry (main.cpp:507-547)
struct Tap { int x0, x1, y0, y1; float fx, fy; };

inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// bilinear_tap, main.cpp:512-531. The bilinear coordinate u*W - 0.5 is a rounded product and a
// rounded difference (the reference's build does not fuse it; the golden vectors pin this at
// image / latent ratios that are not powers of two, where the two forms differ).
inline Tap tap_of(const OrLevel& L, float u, float v) {
    Tap t;
    if (L.nearest) {
        const float x = u * (float)L.W, y = v * (float)L.H;
        const int ix = (int)floorf(x), iy = (int)floorf(y);
        t.fx = x - (float)ix; t.fy = y - (float)iy;
        t.x0 = t.x1 = clampi(ix, 0, L.W - 1);
        t.y0 = t.y1 = clampi(iy, 0, L.H - 1);
        return t;
    }
    const float x = u * (float)L.W - 0.5f, y = v * (float)L.H - 0.5f;
    const int x0 = (int)floorf(x), y0 = (int)floorf(y);
    t.fx = x - (float)x0; t.fy = y - (float)y0;
    t.x0 = clampi(x0, 0, L.W - 1); t.x1 = clampi(x0 + 1, 0, L.W - 1);
    t.y0 = clampi(y0, 0, L.H - 1); t.y1 = clampi(y0 + 1, 0, L.H - 1);
    return t;
}

// bilinear blend weights, main.cpp:543-544
struct Blend { float w00, w10, w01, w11; };
inline Blend blend_of(const Tap& t) {
    Blend b;
    b.w00 = (1.0f - t.fx) * (1.0f - t.fy); b.w10 = t.fx * (1.0f - t.fy);
    b.w01 = (1.0f - t.fx) * t.fy;          b.w11 = t.fx * t.fy;
    return b;
}
// one blended channel, main.cpp:546: w00*a + w10*b + w01*c + w11*d with GCC's contraction
inline float blend(const Blend& b, float a, float bb, float c, float d) {
    return fmaf(b.w11, d, fmaf(b.w01, c, fmaf(b.w00, a, b.w10 * bb)));
}

// sample_latent, main.cpp:533-547 (z = the level's base pointer)
inline void sample(const OrLevel& L, const float* z, const Tap& t, float* out) {
    const float* a = z + ((size_t)t.y0 * L.W + t.x0) * L.C;
    if (L.nearest) { for (int k = 0; k < L.C; k++) out[k] = a[k]; return; }
    const float* b = z + ((size_t)t.y0 * L.W + t.x1) * L.C;
    const float* c = z + ((size_t)t.y1 * L.W + t.x0) * L.C;
    const float* d = z + ((size_t)t.y1 * L.W + t.x1) * L.C;
    const Blend w = blend_of(t);
    for (int k = 0; k < L.C; k++) out[k] = blend(w, a[k], b[k], c[k], d[k]);
}

// Decoder::features + PosEnc::encode, main.cpp:1593-1608, 1687-1702
inline void features(const OrModel& m, const float* z, int px, int py, float* f) {
    const float u = ((float)px + 0.5f) / (float)m.W, v = ((float)py + 0.5f) / (float)m.H;
    const Tap t0 = tap_of(m.lv[0], u, v);
    sample(m.lv[0], z + m.lv[0].off, t0, f);
    int k = m.lv[0].C;
    Tap t1 = t0;
    for (int l = 1; l < m.nlev; l++) {
        const Tap tl = tap_of(m.lv[l], u, v);
        if (l == 1) t1 = tl;
        sample(m.lv[l], z + m.lv[l].off, tl, f + k);
        k += m.lv[l].C;
    }
    for (int q = 0; q < m.npos; q++) {
        if (m.pos[q] == 0) { f[k++] = fmaf(u, 2.0f, -1.0f); f[k++] = fmaf(v, 2.0f, -1.0f); }
        else { f[k++] = fmaf(t1.fx, 2.0f, -1.0f); f[k++] = fmaf(t1.fy, 2.0f, -1.0f); }
    }
}

// ------------------------------------------------------------------ MLP (main.cpp:549-627)
inline float activate(float x, float leak) { return x > 0 ? x : leak * x; }   // main.cpp:560

// mlp_forward, main.cpp:603-627: per unit s = b[j], then s += w[j][i] * a[i] for i ascending
// (one fused multiply-add per term in the reference's build).
inline void mlp_forward(const OrModel& m, const float* p, const float* in, float* out) {
    float bufA[OR_MAXH], bufB[OR_MAXH];
    const float* cur = in;
    int ncur = m.nin;
    float* nxt = bufA;
    for (int l = 0; l < m.nhidden; l++) {
        const int nh = m.hidden[l];
        const float* W = p; const float* b = W + (size_t)nh * ncur;
        for (int j = 0; j < nh; j++) {
            float s = b[j]; const float* w = W + (size_t)j * ncur;
            for (int i = 0; i < ncur; i++) s = fmaf(w[i], cur[i], s);
            nxt[j] = activate(s, m.leak);
        }
        p = b + nh; cur = nxt; ncur = nh;
        nxt = (nxt == bufA) ? bufB : bufA;
    }
    const float* W = p; const float* b = W + (size_t)m.nout * ncur;
    for (int j = 0; j < m.nout; j++) {
        float s = b[j]; const float* w = W + (size_t)j * ncur;
        for (int i = 0; i < ncur; i++) s = fmaf(w[i], cur[i], s);
        out[j] = m.clamp_out ? std::min(1.0f, std::max(0.0f, s + 0.5f)) : 1.0f / (1.0f + expf(-s));
    }
}

inline long long nparams(const OrModel& m) {   // MLP::count, main.cpp:576-580
    long long n = 0; int in = m.nin;
    for (int l = 0; l < m.nhidden; l++) { n += (long long)m.hidden[l] * in + m.hidden[l]; in = m.hidden[l]; }
    return n + (long long)m.nout * in + m.nout;
}
inline long long nzof(const OrModel& m) {
    long long n = 0;
    for (int l = 0; l < m.nlev; l++) n += (long long)m.lv[l].W * m.lv[l].H * m.lv[l].C;
    return n;
}

// Decoder::decode_err's per-pixel term, main.cpp:1731-1732 (float, fused)
inline float pixel_err_f(const OrModel& m, const float* out, const float* t) {
    float e = 0;
    for (int c = 0; c < m.nout; c++) { const float d = out[c] - t[c]; e = fmaf(m.cw[c], d * d, e); }
    return e;
}
// loss_subset's per-pixel terms, main.cpp:1747: float products added into a double
inline void pixel_err_d(const OrModel& m, const float* out, const float* t, double& s) {
    for (int c = 0; c < m.nout; c++) { const float d = out[c] - t[c]; s += (double)(m.cw[c] * (d * d)); }
}

inline double loss_subset(const OrModel& m, const float* p, const float* z, const float* tgt, const int* idx, int n) {
    double s = 0;   // main.cpp:1739-1750
    float f[OR_MAXH], out[OR_MAX_OUT];
    for (int j = 0; j < n; j++) {
        const int i = idx[j];
        features(m, z, i % m.W, i / m.W, f);
        mlp_forward(m, p, f, out);
        pixel_err_d(m, out, tgt + (size_t)i * m.nout, s);
    }
    return s / (3.0 * m.wsum * n);
}

// ------------------------------------------------------------------ DCT (main.cpp:657-1032)
// DCT_BASIS_BITS and DCT_AK_BITS hold the double-precision values rounded once to float; they
// are rebuilt here from their definitions (alpha(u) cos(pi (2x+1) u / 16); 1 / g_k with
// g_k = (14/64) 2^(0.6 k)) and the known-answer tests check every bit pattern.
struct DctTables {
    float basis[64];   // [u * 8 + x]
    float ak[16];
    int zigzag[64];
    DctTables() {
        for (int u = 0; u < 8; u++)
            for (int x = 0; x < 8; x++) {
                const double a = u == 0 ? std::sqrt(1.0 / 8.0) : std::sqrt(2.0 / 8.0);
                basis[u * 8 + x] = (float)(a * std::cos(3.14159265358979323846 * (2 * x + 1) * u / 16.0));
            }
        for (int k = 0; k < 16; k++) ak[k] = (float)(1.0 / ((14.0 / 64.0) * std::pow(2.0, 0.6 * k)));
        // zigzag: anti-diagonals s = u + v, even s walked with u decreasing, odd s with u increasing
        int n = 0;
        for (int s = 0; s < 15; s++) {
            const int ulo = std::max(0, s - 7), uhi = std::min(7, s);
            if (s & 1) for (int u = ulo; u <= uhi; u++) zigzag[n++] = u * 8 + (s - u);
            else for (int u = uhi; u >= ulo; u--) zigzag[n++] = u * 8 + (s - u);
        }
    }
};
const DctTables& dct_tables() { static const DctTables T; return T; }

const int JPEG_K1[8][8] = {   // JPEG Annex K Table K.1 (luminance), rows = vertical frequency
    { 16, 11, 10, 16, 24, 40, 51, 61 }, { 12, 12, 14, 19, 26, 58, 60, 55 },
    { 14, 13, 16, 24, 40, 57, 69, 56 }, { 14, 17, 22, 29, 51, 87, 80, 62 },
    { 18, 22, 37, 56, 68, 109, 103, 77 }, { 24, 35, 55, 64, 81, 104, 113, 92 },
    { 49, 64, 78, 87, 103, 121, 120, 101 }, { 72, 92, 95, 98, 112, 100, 103, 99 },
};

inline float dct_clampf(float v, float lo, float hi) { if (!(v >= lo)) return lo; if (v > hi) return hi; return v; }   // main.cpp:798
inline bool first_order(int u, int v) { return (u == 1 && v == 0) || (u == 0 && v == 1); }
inline int floor_log2(unsigned v) { int k = 0; while (v >>= 1) k++; return k; }
inline int c_run(int r) { return 16 * (2 * floor_log2((unsigned)(r + 1)) + 1); }   // main.cpp:832
inline int c_mag(int m) { return 16 * (2 * floor_log2((unsigned)m) + 1); }         // main.cpp:833
inline int lo_weight(int tok, int p, int lo16) { return p <= 2 ? (tok * lo16 + 8) >> 4 : tok; }   // main.cpp:834

inline int quant_dc(float d, int S) { return (int)dct_clampf(nearbyintf(d / (float)S), -1024.0f, 1024.0f); }   // main.cpp:800
inline float dequant_dc(int q, int S) { return (float)q * (float)S; }
inline int quant_ac(float d, int L, int u, int v, bool dz) {   // main.cpp:807-814
    if (!dz || first_order(u, v)) return (int)dct_clampf(roundf(d / (float)L), -1024.0f, 1024.0f);
    const float s = fabsf(d), tau = 0.5f * (float)L;
    if (s <= tau) return 0;
    const float qf = (s - tau) / (float)L;
    const int q = (int)dct_clampf(floorf(qf + 0.5f), 0.0f, 1024.0f);
    return d < 0.0f ? -q : q;
}
inline float dequant_ac(int q, int L, int u, int v, bool dz) {   // main.cpp:815-821
    if (!dz || first_order(u, v)) return (float)q * (float)L;
    if (q == 0) return 0.0f;
    const float tau = 0.5f * (float)L;
    const float mag = tau + (float)std::abs(q) * (float)L;
    return q < 0 ? -mag : mag;
}
// dct_fwd8 / dct_inv8, main.cpp:783-796: w[x*8+y], C[u*8+v]; sequential sums from 0, strict
void fwd8(const float* w, float* C) {
    const float* B = dct_tables().basis;
    float T[64];
    for (int x = 0; x < 8; x++)
        for (int v = 0; v < 8; v++) { float s = 0.0f; for (int y = 0; y < 8; y++) s += w[x * 8 + y] * B[v * 8 + y]; T[x * 8 + v] = s; }
    for (int u = 0; u < 8; u++)
        for (int v = 0; v < 8; v++) { float s = 0.0f; for (int x = 0; x < 8; x++) s += T[x * 8 + v] * B[u * 8 + x]; C[u * 8 + v] = s; }
}
void inv8(const float* C, float* w) {
    const float* B = dct_tables().basis;
    float T[64];
    for (int x = 0; x < 8; x++)
        for (int v = 0; v < 8; v++) { float s = 0.0f; for (int u = 0; u < 8; u++) s += B[u * 8 + x] * C[u * 8 + v]; T[x * 8 + v] = s; }
    for (int x = 0; x < 8; x++)
        for (int y = 0; y < 8; y++) { float s = 0.0f; for (int v = 0; v < 8; v++) s += B[v * 8 + y] * T[x * 8 + v]; w[x * 8 + y] = s; }
}
int block_bits(const int16_t* sym, int lo16) {   // dct_block_bits, main.cpp:835-845
    const int* zz = dct_tables().zigzag;
    int bits = 0, run = 0, lnz = 0;
    for (int p = 1; p < 64; p++) {
        const int q = sym[zz[p]];
        if (q == 0) { run++; continue; }
        bits += lo_weight(c_run(run) + c_mag(std::min(256, std::abs(q))) + 16, p, lo16);
        lnz = p; run = 0;
    }
    if (lnz < 63) bits += 32;
    return bits;
}
int truncate_block(const float* Cf, const int* st, float lam16, int lo16, bool dz, int16_t* sym) {   // main.cpp:850-867
    const int* zz = dct_tables().zigzag;
    int ntrunc = 0, next = 64;
    for (int p = 63; p >= 1; p--) {
        const int k = zz[p], q = sym[k];
        if (q == 0) continue;
        int prev = 0;
        for (int j = p - 1; j >= 1; j--) if (sym[zz[j]] != 0) { prev = j; break; }
        const int r1 = p - prev - 1;
        const int token = lo_weight(c_run(r1) + c_mag(std::min(256, std::abs(q))) + 16, p, lo16);
        const int saved = next == 64 ? token - (p == 63 ? 32 : 0) : token + c_run(next - p - 1) - c_run(next - p - 1 + r1 + 1);
        const float v = dequant_ac(q, st[k], k / 8, k % 8, dz), c = Cf[k];
        const float dD = c * c - (c - v) * (c - v);
        if (dD < lam16 * (float)saved) { sym[k] = 0; ntrunc++; }
        else next = p;
    }
    return ntrunc;
}
int quantize_block(const float* Cf, const int* st, int dc_step, float lam16, int lo16, bool dz, bool with_bits,
                   int16_t* sym, int* ntrunc, int* nz_before) {   // main.cpp:871-881
    for (int k = 0; k < 64; k++) sym[k] = (int16_t)(k == 0 ? quant_dc(Cf[0], dc_step) : quant_ac(Cf[k], st[k], k / 8, k % 8, dz));
    int nt = 0, nz = 0;
    if (lam16 > 0.0f) {
        for (int k = 1; k < 64; k++) if (sym[k] != 0) nz++;
        nt = truncate_block(Cf, st, lam16, lo16, dz, sym);
    }
    if (ntrunc) *ntrunc = nt;
    if (nz_before) *nz_before = nz;
    return with_bits ? block_bits(sym, lo16) : 0;
}
inline size_t lvl0_index(const OrLevel& L0, int bx, int by, int x, int y, int c) {
    return ((size_t)(by * 8 + y) * L0.W + (bx * 8 + x)) * L0.C + c;
}
// dct_recon_block, main.cpp:899-915 (zq = level-0 base pointer); returns clamped texels
int recon_block(const OrDct& Q, const OrLevel& L0, size_t b, int c, float* zq) {
    float Cf[64], w[64];
    const int16_t* sy = Q.sym + (b * Q.C + c) * 64;
    const int* st = Q.step + ((size_t)c * 16 + Q.code[b * Q.C + c]) * 64;
    for (int k = 0; k < 64; k++) Cf[k] = k == 0 ? dequant_dc(sy[0], Q.dc_step) : dequant_ac(sy[k], st[k], k / 8, k % 8, Q.deadzone != 0);
    inv8(Cf, w);
    const int bx = (int)(b % Q.BW), by = (int)(b / Q.BW);
    int nclamp = 0;
    for (int y = 0; y < 8; y++)
        for (int x = 0; x < 8; x++) {
            const float raw = w[y * 8 + x] / 32.0f - 1.0f;
            const float v = dct_clampf(raw, -1.0f, 1.0f);
            if (v != raw) nclamp++;
            zq[lvl0_index(L0, bx, by, x, y, c)] = v;
        }
    return nclamp;
}

// ------------------------------------------------------------------ QES (main.cpp:446-495)
inline int qes_index(float v, float lo, float range, int levels) {
    const float r = nearbyintf(((v - lo) / range) * (float)levels);
    if (!(r == r)) return 0;   // NaN: the index the device's saturating conversion gives
    return r <= 0.0f ? 0 : (r >= (float)levels ? levels : (int)r);
}

// ------------------------------------------------------------------ QAT (main.cpp:2054-2065)
inline int qat_index(float v, int bits) {
    const int levels = (1 << bits) - 1;
    const int k = (int)std::lround((v + 1.0f) * 0.5f * (float)levels);
    return std::max(0, std::min(levels, k));
}

}   // namespace

// ==================================================================== extern "C" API
extern "C" {

uint64_t or_mix64(uint64_t x) { return mix64(x); }
uint64_t or_noise_key(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index) { return noise_key(seed, stream, step, pair, index); }
uint32_t or_noise_u32(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index) { return (uint32_t)(noise_key(seed, stream, step, pair, index) >> 32); }
uint32_t or_noise_uniform(uint32_t u, uint32_t n) { return (uint32_t)(((uint64_t)u * (uint64_t)n) >> 32); }
float or_gauss(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index) { return gauss(seed, stream, step, pair, index); }
void or_gauss_fill(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair, uint64_t index0, long long n, float* out) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < n; i++) out[i] = gauss(seed, stream, step, pair, index0 + (uint64_t)i);
}
float or_gauss_radius(uint32_t k1) { return radius_of(k1); }
float or_gauss_cosine(uint32_t k2) { return cosine_of(k2); }
void or_gauss_factors(uint32_t k0, long long n, float* rad, float* cosv) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < n; i++) { rad[i] = radius_of(k0 + (uint32_t)i); cosv[i] = cosine_of(k0 + (uint32_t)i); }
}

long long or_model_nparams(const OrModel* m) { return nparams(*m); }
long long or_model_nz(const OrModel* m) { return nzof(*m); }
void or_tap(const OrLevel* L, float u, float v, int* r, float* f) {
    const Tap t = tap_of(*L, u, v);
    r[0] = t.x0; r[1] = t.x1; r[2] = t.y0; r[3] = t.y1; f[0] = t.fx; f[1] = t.fy;
}
void or_features(const OrModel* m, const float* z, int px, int py, float* f) { features(*m, z, px, py, f); }
void or_mlp_forward(const OrModel* m, const float* p, const float* in, float* out) { mlp_forward(*m, p, in, out); }

// Decoder::decode_full, main.cpp:1712-1718
void or_decode_full(const OrModel* mp, const float* p, const float* z, float* img) {
    const OrModel& m = *mp;
#pragma omp parallel for schedule(static)
    for (int y = 0; y < m.H; y++) {
        float f[OR_MAXH];
        for (int x = 0; x < m.W; x++) {
            features(m, z, x, y, f);
            mlp_forward(m, p, f, img + ((size_t)y * m.W + x) * m.nout);
        }
    }
}
// Decoder::decode_err, main.cpp:1722-1735
void or_decode_err(const OrModel* mp, const float* p, const float* z, const float* tgt, float* err) {
    const OrModel& m = *mp;
#pragma omp parallel for schedule(static)
    for (int y = 0; y < m.H; y++) {
        float f[OR_MAXH], out[OR_MAX_OUT];
        for (int x = 0; x < m.W; x++) {
            const size_t i = (size_t)y * m.W + x;
            features(m, z, x, y, f);
            mlp_forward(m, p, f, out);
            err[i] = pixel_err_f(m, out, tgt + i * m.nout);
        }
    }
}
double or_loss_subset(const OrModel* m, const float* p, const float* z, const float* tgt, const int* idx, int n) {
    return loss_subset(*m, p, z, tgt, idx, n);
}

// MlpTrainer::draw_batch with --rng hash, main.cpp:1825-1833
void or_draw_batch(uint64_t seed, int it, int M, int npix, int* idx) {
    for (int s = 0; s < M; s++)
        idx[s] = (int)or_noise_uniform((uint32_t)(noise_key(seed, NS_BATCH_PIX, (uint32_t)it, 0, (uint64_t)s) >> 32), (uint32_t)npix);
}

// The pair evaluations of MlpTrainer::step, main.cpp:1839-1861: member +/- of pair i has the
// weights p0 +/- sigma * eps_i (one fused operation each in the reference's build).
void or_mlp_es_eval(const OrModel* mp, const float* p0, const float* z, const float* tgt, uint64_t seed, int it,
                    float sigma, int N, const int* idx, int M, double* dl, double* lsum, double* lp_out, double* lm_out) {
    const OrModel& m = *mp;
    const long long P = nparams(m);
#pragma omp parallel
    {
        std::vector<float> pp(P), pm(P);
#pragma omp for schedule(dynamic)
        for (int i = 0; i < N; i++) {
            for (long long k = 0; k < P; k++) {
                const float e = gauss(seed, NS_MLP, (uint32_t)it, (uint32_t)i, (uint64_t)k);
                pp[k] = fmaf(sigma, e, p0[k]);
                pm[k] = fmaf(-sigma, e, p0[k]);
            }
            const double lp = loss_subset(m, pp.data(), z, tgt, idx, M);
            const double lm = loss_subset(m, pm.data(), z, tgt, idx, M);
            dl[i] = lp - lm; lsum[i] = 0.5 * (lp + lm);
            if (lp_out) lp_out[i] = lp;
            if (lm_out) lm_out[i] = lm;
        }
    }
}
// The gradient of MlpTrainer::step, main.cpp:1867-1873: pairs in order, one fused add per pair.
void or_mlp_es_grad(long long P, int N, uint64_t seed, int it, float sigma, const double* dl, float* grad) {
    const float scale = 1.0f / (2.0f * (float)N * sigma);
#pragma omp parallel for schedule(static)
    for (long long k = 0; k < P; k++) {
        float g = 0.0f;
        for (int i = 0; i < N; i++) g = fmaf((float)dl[i] * scale, gauss(seed, NS_MLP, (uint32_t)it, (uint32_t)i, (uint64_t)k), g);
        grad[k] = g;
    }
}
// Adam::step, main.cpp:1799-1809; t is the step count after the increment.
void or_adam(float* theta, const float* g, float* m, float* v, long long n, float lr, int t) {
    const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    const float c1 = 1.0f - powf(b1, (float)t), c2 = 1.0f - powf(b2, (float)t);
    const float ob1 = 1.0f - b1, ob2 = 1.0f - b2;
    for (long long i = 0; i < n; i++) {
        m[i] = fmaf(b1, m[i], ob1 * g[i]);
        v[i] = fmaf(b2, v[i], (ob2 * g[i]) * g[i]);
        const float mh = m[i] / c1, vh = v[i] / c2;
        theta[i] = theta[i] - (lr * mh) / (sqrtf(vh) + eps);
    }
}
// MlpTrainer::step_fd, main.cpp:1890-1920 (per weight: float-realized steps)
void or_mlp_fd_eval(const OrModel* mp, const float* p0, const float* z, const float* tgt, float h,
                    const int* idx, int M, double* dl, double* hh, double* l0) {
    const OrModel& m = *mp;
    const long long P = nparams(m);
    if (l0) *l0 = loss_subset(m, p0, z, tgt, idx, M);
#pragma omp parallel
    {
        std::vector<float> pw(p0, p0 + P);
#pragma omp for schedule(dynamic, 16)
        for (long long j = 0; j < P; j++) {
            const float orig = pw[j], wp = orig + h, wm = orig - h;
            pw[j] = wp; const double lp = loss_subset(m, pw.data(), z, tgt, idx, M);
            pw[j] = wm; const double lm = loss_subset(m, pw.data(), z, tgt, idx, M);
            pw[j] = orig;
            dl[j] = lp - lm; hh[j] = (double)wp - (double)wm;
        }
    }
}
void or_fd_grad(long long P, const double* dl, const double* hh, float* grad) {
    for (long long j = 0; j < P; j++) grad[j] = (float)(dl[j] / hh[j]);
}

// LatentTrainer::step_impl, main.cpp:1974-2044, and dct_rate_pass, main.cpp:1935-1952.
// One pair's mse scatter (main.cpp:2011-2037): every pixel in raster order adds its loss difference d to
// each distinct tap texel of every active level, then grad += (dtex * scale) * eps per texel channel.
static void lat_scatter_pair(const OrModel& m, unsigned active_mask, const float* d, const float* eps, float scale,
                             std::vector<float>& dtex, float* grad) {
    for (int l = 0; l < m.nlev; l++) {
        if (!((active_mask >> l) & 1u)) continue;
        const OrLevel& L = m.lv[l];
        const size_t ntex = (size_t)L.W * L.H;
        std::fill(dtex.begin(), dtex.begin() + ntex, 0.0f);
        for (int py = 0; py < m.H; py++) {
            const float v = ((float)py + 0.5f) / (float)m.H;
            for (int px = 0; px < m.W; px++) {
                const float u = ((float)px + 0.5f) / (float)m.W;
                const float dp = d[(size_t)py * m.W + px];
                const Tap t = tap_of(L, u, v);
                dtex[(size_t)t.y0 * L.W + t.x0] += dp;
                if (t.x1 != t.x0) dtex[(size_t)t.y0 * L.W + t.x1] += dp;
                if (t.y1 != t.y0) {
                    dtex[(size_t)t.y1 * L.W + t.x0] += dp;
                    if (t.x1 != t.x0) dtex[(size_t)t.y1 * L.W + t.x1] += dp;
                }
            }
        }
        for (size_t ti = 0; ti < ntex; ti++) {
            const float w = dtex[ti] * scale;
            const size_t base = (size_t)L.off + ti * L.C;
            for (int c = 0; c < L.C; c++) grad[base + c] = fmaf(w, eps[base + c], grad[base + c]);
        }
    }
}

static size_t max_texels(const OrModel& m) {
    size_t maxtex = 0;
    for (int l = 0; l < m.nlev; l++) maxtex = std::max(maxtex, (size_t)m.lv[l].W * m.lv[l].H);
    return maxtex;
}

// The latent gradient of K pairs from given per-pixel loss differences dpix [K][W*H] and Gaussians
// eps [K][nz] (the scatter of or_lat_grad alone, without a rate term)
void or_lat_scatter(const OrModel* mp, const float* eps, const float* dpix, int K, unsigned active_mask, float sigma,
                    float* grad) {
    const OrModel& m = *mp;
    const size_t n = (size_t)nzof(m), npix = (size_t)m.W * m.H;
    std::vector<float> dtex(max_texels(m));
    std::fill(grad, grad + n, 0.0f);
    const float scale = 1.0f / (2.0f * (float)K * sigma);
    for (int k = 0; k < K; k++) lat_scatter_pair(m, active_mask, dpix + (size_t)k * npix, eps + (size_t)k * n, scale, dtex, grad);
}

void or_lat_grad(const OrModel* mp, const float* p, const float* zdec, const float* zshadow, const float* tgt,
                 uint64_t seed, int step_no, float sigma, int K, unsigned active_mask,
                 const OrDct* dct, float rate_scale, float* grad, float* dpix, int32_t* dbits_last, int* hits) {
    const OrModel& m = *mp;
    const size_t n = (size_t)nzof(m), npix = (size_t)m.W * m.H;
    std::vector<float> eps(n), zp(n), zm(n), ep(npix), em(npix), d(npix);
    std::vector<float> dtex(max_texels(m));
    std::fill(grad, grad + n, 0.0f);
    const float inv_px = 1.0f / (3.0f * m.wsum * (float)m.W * (float)m.H);
    const float sg = sigma;
    int nhits = 0;
    for (int k = 0; k < K; k++) {
        for (int l = 0; l < m.nlev; l++) {
            const OrLevel& L = m.lv[l];
            const size_t o = (size_t)L.off, sz = (size_t)L.W * L.H * L.C;
            const bool active = (active_mask >> l) & 1u;
            for (size_t i = o; i < o + sz; i++) {
                if (active) {
                    eps[i] = gauss(seed, NS_LAT, (uint32_t)step_no, (uint32_t)k, (uint64_t)i);
                    zp[i] = fmaf(sg, eps[i], zdec[i]);
                    zm[i] = fmaf(-sg, eps[i], zdec[i]);
                } else { eps[i] = 0.0f; zp[i] = zdec[i]; zm[i] = zdec[i]; }
            }
        }
        or_decode_err(mp, p, zp.data(), tgt, ep.data());
        or_decode_err(mp, p, zm.data(), tgt, em.data());
        for (size_t i = 0; i < npix; i++) d[i] = (ep[i] - em[i]) * inv_px;
        if (dpix) std::copy(d.begin(), d.end(), dpix + (size_t)k * npix);
        lat_scatter_pair(m, active_mask, d.data(), eps.data(), 1.0f / (2.0f * (float)K * sg), dtex, grad);
        if (dct) {   // the rate pass of this pair, after the mse scatter
            const OrLevel& L0 = m.lv[0];
            const size_t nbc = (size_t)dct->BW * dct->BH * dct->C;
            std::vector<int32_t> db(nbc);
            or_dct_rate_pair(dct, &L0, zshadow + L0.off, eps.data() + L0.off, sg, db.data());
            for (size_t i = 0; i < nbc; i++) if (db[i] != 0) nhits++;
            const float scale = 1.0f / (2.0f * (float)K * sg);
            for (int ty = 0; ty < L0.H; ty++)
                for (int tx = 0; tx < L0.W; tx++) {
                    const size_t b = (size_t)(ty / 8) * dct->BW + (size_t)(tx / 8);
                    const size_t base = (size_t)L0.off + ((size_t)ty * L0.W + tx) * L0.C;
                    for (int c = 0; c < L0.C; c++)
                        grad[base + c] = fmaf((rate_scale * (float)db[b * dct->C + c]) * scale, eps[base + c], grad[base + c]);
                }
            if (dbits_last && k == K - 1) memcpy(dbits_last, db.data(), nbc * sizeof(int32_t));
        }
    }
    if (hits) *hits = nhits;
}

// QAT_GRID, main.cpp:2054-2057
void or_qat_grid(float* grid) {
    memset(grid, 0, sizeof(float) * 9 * 257);
    for (int b = 1; b <= 8; b++) {
        const int levels = (1 << b) - 1;
        for (int k = 0; k <= levels; k++) grid[b * 257 + k] = -1.0f + (2.0f * (float)k) / (float)levels;
    }
}
int or_qat_index(float v, int bits) { return qat_index(v, bits); }

// qat_search, main.cpp:2088-2139 (on the decode buffer; texels independent)
void or_qat_search(const OrModel* mp, const float* p, float* z, const float* tgt, const int* ch_bits, const float* grid) {
    const OrModel& m = *mp;
    const OrLevel& L = m.lv[0];
    const int nin = m.nin, nc = m.nout;
    std::vector<int> xb(L.W, m.W), xe(L.W, 0), yb(L.H, m.H), ye(L.H, 0);
    for (int px = 0; px < m.W; px++) { const int t = tap_of(L, ((float)px + 0.5f) / (float)m.W, 0.5f).x0; xb[t] = std::min(xb[t], px); xe[t] = std::max(xe[t], px + 1); }
    for (int py = 0; py < m.H; py++) { const int t = tap_of(L, 0.5f, ((float)py + 0.5f) / (float)m.H).y0; yb[t] = std::min(yb[t], py); ye[t] = std::max(ye[t], py + 1); }
#pragma omp parallel
    {
        std::vector<float> feat;
#pragma omp for schedule(dynamic)
        for (int ty = 0; ty < L.H; ty++)
            for (int tx = 0; tx < L.W; tx++) {
                const int x0 = xb[tx], x1 = xe[tx], y0 = yb[ty], y1 = ye[ty];
                if (x0 >= x1 || y0 >= y1) continue;
                const int npx = (x1 - x0) * (y1 - y0);
                feat.resize((size_t)npx * nin);
                { int j = 0; for (int py = y0; py < y1; py++) for (int px = x0; px < x1; px++, j++) features(m, z, px, py, &feat[(size_t)j * nin]); }
                float* zt = z + L.off + ((size_t)ty * L.W + tx) * L.C;
                for (int c = 0; c < L.C; c++) {
                    const int bits = ch_bits[c], levels = (1 << bits) - 1;
                    const float* g = grid + bits * 257;
                    auto cell_loss = [&](float val) {
                        double sum = 0; int j = 0;
                        for (int py = y0; py < y1; py++)
                            for (int px = x0; px < x1; px++, j++) {
                                float* f = &feat[(size_t)j * nin]; f[c] = val;
                                float out[OR_MAX_OUT];
                                mlp_forward(m, p, f, out);
                                pixel_err_d(m, out, tgt + ((size_t)py * m.W + px) * nc, sum);
                            }
                        return sum;
                    };
                    int best_k = qat_index(zt[c], bits);
                    double best = cell_loss(g[best_k]);
                    for (int k = 0; k <= levels; k++) {
                        if (k == best_k) continue;
                        const double sk = cell_loss(g[k]);
                        if (sk < best) { best = sk; best_k = k; }
                    }
                    zt[c] = g[best_k];
                    for (int j = 0; j < npx; j++) feat[(size_t)j * nin + c] = g[best_k];
                }
            }
    }
}

int or_qes_index(float v, float lo, float range, int levels) { return qes_index(v, lo, range, levels); }
// qes_fit, main.cpp:455-464 (z = the level's base pointer)
void or_qes_fit(const OrLevel* L, const float* z, int bits, float* lo, float* hi, float* range, float* grid) {
    const int levels = (1 << bits) - 1, C = L->C;
    const size_t n = (size_t)L->W * L->H * C;
    for (int c = 0; c < C; c++) { lo[c] = 1e30f; hi[c] = -1e30f; }
    for (size_t i = 0; i < n; i++) { const int c = (int)(i % C); lo[c] = std::min(lo[c], z[i]); hi[c] = std::max(hi[c], z[i]); }
    for (int c = 0; c < C; c++) {
        range[c] = std::max(hi[c] - lo[c], 1e-6f);
        for (int k = 0; k <= levels; k++) grid[(size_t)c * (levels + 1) + k] = lo[c] + ((float)k / (float)levels) * range[c];
    }
}
// qes_snap_level, main.cpp:485-495
long long or_qes_snap_level(const OrLevel* L, int bits, const float* lo, const float* hi, const float* range,
                            const float* grid, float* z, float* zq, int clamp) {
    const int levels = (1 << bits) - 1, C = L->C;
    const size_t n = (size_t)L->W * L->H * C;
    long long changed = 0;
    for (size_t i = 0; i < n; i++) {
        const int c = (int)(i % C);
        float v = z[i];
        if (clamp) { v = std::min(std::max(v, lo[c]), hi[c]); z[i] = v; }
        const float s = grid[(size_t)c * (levels + 1) + qes_index(v, lo[c], range[c], levels)];
        if (s != zq[i]) { zq[i] = s; changed++; }
    }
    return changed;
}

void or_dct_tables(float* basis, int* zigzag, float* ak) {
    const DctTables& T = dct_tables();
    if (basis) memcpy(basis, T.basis, sizeof(T.basis));
    if (zigzag) memcpy(zigzag, T.zigzag, sizeof(T.zigzag));
    if (ak) memcpy(ak, T.ak, sizeof(T.ak));
}
float or_dct_quality_scale(int q) {   // main.cpp:747-752
    q = std::max(1, std::min(100, q));
    float S = q < 50 ? 5000.0f / (float)q : 200.0f - 2.0f * (float)q;
    S *= (1.0f / 100.0f);
    return S;
}
// dct_build_steps_scaled at N = 8 (sx = 1: the table entry itself), main.cpp:758-775
void or_dct_build_steps_scaled(int q, float level_scale, int dc_step, int* out) {
    for (int u = 0; u < 8; u++)
        for (int v = 0; v < 8; v++) {
            if (u == 0 && v == 0) { out[0] = dc_step; continue; }
            if (q >= 100) { out[u * 8 + v] = 1; continue; }
            const float base = (float)JPEG_K1[u][v];
            float sf = base * level_scale + 0.5f;
            if (!(sf >= 1.0f)) sf = 1.0f;
            if (sf > 1048576.0f) sf = 1048576.0f;
            out[u * 8 + v] = std::max(1, (int)sf);
        }
}
void or_dct_build_steps(int q, int dc_step, int* out) {   // main.cpp:777-779
    const float S = or_dct_quality_scale(q);
    for (int k = 0; k < 16; k++) or_dct_build_steps_scaled(q, S * dct_tables().ak[k], dc_step, out + (size_t)k * 64);
}
void or_dct_fwd8(const float* w, float* C) { fwd8(w, C); }
void or_dct_inv8(const float* C, float* w) { inv8(C, w); }
int or_dct_quant_dc(float d, int S) { return quant_dc(d, S); }
float or_dct_dequant_dc(int q, int S) { return dequant_dc(q, S); }
int or_dct_quant_ac(float d, int L, int u, int v, int dz) { return quant_ac(d, L, u, v, dz != 0); }
float or_dct_dequant_ac(int q, int L, int u, int v, int dz) { return dequant_ac(q, L, u, v, dz != 0); }
int or_dct_c_run(int r) { return c_run(r); }
int or_dct_c_mag(int m) { return c_mag(m); }
int or_dct_block_bits(const int16_t* sym, int lo16) { return block_bits(sym, lo16); }
int or_dct_quantize_block(const float* Cf, const int* st, int dc_step, float lam16, int lo16, int dz, int with_bits,
                          int16_t* sym, int* ntrunc, int* nz_before) {
    return quantize_block(Cf, st, dc_step, lam16, lo16, dz != 0, with_bits != 0, sym, ntrunc, nz_before);
}
int or_dct_code_of_gain(double g) {   // main.cpp:980-985
    const double gf = 14.0 / 64.0;
    if (!(g > gf)) g = gf;
    const long k = std::lround(std::log2(g / gf) / 0.6);
    return (int)std::max(0L, std::min(15L, k));
}
double or_dct_gain_of_code(int k) { return (14.0 / 64.0) * std::pow(2.0, 0.6 * k); }
void or_dct_clamp_level0(const OrLevel* L0, float* z) {   // main.cpp:974-976
    const size_t n = (size_t)L0->W * L0->H * L0->C;
    for (size_t i = 0; i < n; i++) z[i] = dct_clampf(z[i], -1.0f, 1.0f);
}
// dct_snap_level0 / dct_snap_block, main.cpp:918-957 (z, zq = level-0 base pointers)
void or_dct_snap_level0(const OrDct* d, const OrLevel* L0, float* z, float* zq, int32_t* bits, long long* counts) {
    const OrDct& Q = *d;
    long long nt_all = 0, nz_all = 0, ncl = 0;
    const size_t nb = (size_t)Q.BW * Q.BH;
    for (size_t b = 0; b < nb; b++)
        for (int c = 0; c < Q.C; c++) {
            float w[64], Cf[64];
            const int bx = (int)(b % Q.BW), by = (int)(b / Q.BW);
            for (int y = 0; y < 8; y++)
                for (int x = 0; x < 8; x++) {
                    const size_t i = lvl0_index(*L0, bx, by, x, y, c);
                    const float s = dct_clampf(z[i], -1.0f, 1.0f);
                    z[i] = s;
                    w[y * 8 + x] = (s + 1.0f) * 32.0f;
                }
            fwd8(w, Cf);
            const int code = Q.code[b * Q.C + c];
            const int* st = Q.step + ((size_t)c * 16 + code) * 64;
            int16_t* sym = Q.sym + (b * Q.C + c) * 64;
            int nt = 0, nz = 0;
            quantize_block(Cf, st, Q.dc_step, Q.lam_t16[code], Q.lo_w16, Q.deadzone != 0, false, sym, &nt, &nz);
            nt_all += nt; nz_all += nz;
            if (bits) bits[b * Q.C + c] = block_bits(sym, Q.lo_w16);
            ncl += recon_block(Q, *L0, b, c, zq);
        }
    if (counts) { counts[0] = nt_all; counts[1] = nz_all; counts[2] = ncl; }
}
void or_dct_recon_level0(const OrDct* d, const OrLevel* L0, float* zq, int32_t* bits) {   // main.cpp:959-972
    const size_t nb = (size_t)d->BW * d->BH;
    for (size_t b = 0; b < nb; b++)
        for (int c = 0; c < d->C; c++) {
            if (bits) bits[b * d->C + c] = block_bits(d->sym + (b * d->C + c) * 64, d->lo_w16);
            recon_block(*d, *L0, b, c, zq);
        }
}
// dct_probe_codes, main.cpp:1001-1032 (features on the decode buffer zdec)
void or_dct_probe_codes(const OrModel* mp, const float* p, const float* zdec, const OrDct* d, uint8_t* code) {
    const OrModel& m = *mp;
    static const int PP[2] = { 2, 5 };
    static const float SJ[5] = { -1.0f, -0.5f, 0.0f, 0.5f, 1.0f };
#pragma omp parallel for schedule(dynamic)
    for (int by = 0; by < d->BH; by++)
        for (int bx = 0; bx < d->BW; bx++)
            for (int c = 0; c < d->C; c++) {
                double acc = 0.0;
                for (int py = 0; py < 2; py++)
                    for (int px = 0; px < 2; px++) {
                        float f[OR_MAXH], out[5][OR_MAX_OUT];
                        features(m, zdec, bx * 8 + PP[px], by * 8 + PP[py], f);
                        for (int j = 0; j < 5; j++) { f[c] = SJ[j]; mlp_forward(m, p, f, out[j]); }
                        for (int j = 0; j < 4; j++) {
                            double ss = 0.0;
                            for (int o = 0; o < m.nout; o++) { const double dd = (double)out[j + 1][o] - (double)out[j][o]; ss += m.cw[o] * dd * dd; }
                            const double g = (255.0 / 16.0) * std::sqrt(ss / m.wsum);
                            acc += g * g;
                        }
                    }
                code[((size_t)by * d->BW + bx) * d->C + c] = (uint8_t)or_dct_code_of_gain(std::sqrt(acc / 16.0));
            }
}
// dct_rate_block for both signs (main.cpp:884-896) over every (block, channel): dbits = bits(+) - bits(-)
void or_dct_rate_pair(const OrDct* d, const OrLevel* L0, const float* z, const float* eps0, float sg, int32_t* dbits) {
    const OrDct& Q = *d;
    const size_t nb = (size_t)Q.BW * Q.BH;
    for (size_t b = 0; b < nb; b++)
        for (int c = 0; c < Q.C; c++) {
            int bb[2];
            const int bx = (int)(b % Q.BW), by = (int)(b / Q.BW);
            const int code = Q.code[b * Q.C + c];
            for (int sgn = 0; sgn < 2; sgn++) {
                float w[64], Cf[64]; int16_t sym[64];
                for (int y = 0; y < 8; y++)
                    for (int x = 0; x < 8; x++) {
                        const size_t i = lvl0_index(*L0, bx, by, x, y, c);
                        const float pert = sg * eps0[i];
                        const float s = dct_clampf(sgn == 0 ? z[i] + pert : z[i] - pert, -1.0f, 1.0f);
                        w[y * 8 + x] = (s + 1.0f) * 32.0f;
                    }
                fwd8(w, Cf);
                bb[sgn] = quantize_block(Cf, Q.step + ((size_t)c * 16 + code) * 64, Q.dc_step, Q.lam_t16[code], Q.lo_w16,
                                         Q.deadzone != 0, true, sym, nullptr, nullptr);
            }
            dbits[b * Q.C + c] = bb[0] - bb[1];
        }
}

// the host branch of --dct-shadow-pull, main.cpp:4142-4146 (the reference's build fuses the update)
void or_shadow_pull(float* z, const float* zq, long long n, float f) {
    for (long long i = 0; i < n; i++) z[i] = fmaf(f, zq[i] - z[i], z[i]);
}

// ntcb_f32_to_f16 / ntcb_f16_to_f32, main.cpp:2427-2455: binary16 with round-half-even
uint16_t or_f32_to_f16(float f, int* overflow) {
    uint32_t u; memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int ex = (int)((u >> 23) & 0xFFu);
    uint32_t man = u & 0x7FFFFFu;
    if (ex == 0xFF) { *overflow = 1; return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u)); }
    const int e = ex - 127 + 15;
    if (e >= 0x1F) { *overflow = 1; return (uint16_t)(sign | 0x7C00u); }
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        const int shift = 14 - e;
        uint32_t half = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1u), mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (half & 1u))) half++;
        return (uint16_t)(sign | half);
    }
    uint32_t half = sign | ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) { half++; if ((half & 0x7C00u) == 0x7C00u) *overflow = 1; }
    return (uint16_t)half;
}
float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const int e = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FFu, u;
    if (e == 0) {
        if (man == 0) u = sign;
        else { int ee = -1; do { ee++; man <<= 1; } while ((man & 0x400u) == 0); u = sign | ((uint32_t)(127 - 15 - ee) << 23) | ((man & 0x3FFu) << 13); }
    } else if (e == 31) u = sign | 0x7F800000u | (man << 13);
    else u = sign | ((uint32_t)(e - 15 + 127) << 23) | (man << 13);
    float f; memcpy(&f, &u, 4); return f;
}
// ntcb_mlp_round_fp16, main.cpp:2472-2481; returns 0 when a weight has no fp16 value
int or_round_fp16(float* p, long long n, long long* changed) {
    long long ch = 0;
    for (long long i = 0; i < n; i++) {
        int ov = 0; const uint16_t h = or_f32_to_f16(p[i], &ov);
        if (ov || !std::isfinite(p[i])) return 0;
        const float r = or_f16_to_f32(h);
        if (r != p[i]) { ch++; p[i] = r; }
    }
    if (changed) *changed = ch;
    return 1;
}
int or_q8_index(float z, float lo, float range, int levels) {   // main.cpp:478-481
    const int qi = (int)std::lround((z - lo) / range * (float)levels);
    return std::max(0, std::min(levels, qi));
}
float or_q8_value(int k, float lo, float range, int levels) { return lo + ((float)k / (float)levels) * range; }   // main.cpp:482

// One iteration of the training loop, main.cpp:4121-4148, CPU branch with --rng hash, without
// --qes / --dct-q (those switch on the host and are exercised through their own functions).
double or_train_iter(const OrModel* mp, const OrTrainCfg* c, OrTrainState* s, const float* tgt, int it, int iters) {
    const OrModel& m = *mp;
    const long long P = nparams(m), nz = nzof(m);
    (void)iters;
    std::vector<int> idx(c->mlp_batch);
    or_draw_batch(c->seed, it, c->mlp_batch, m.W * m.H, idx.data());
    std::vector<float> grad(P);
    double loss;
    if (it >= c->fd_from) {
        if (it == c->fd_from) { std::fill(s->wm, s->wm + P, 0.0f); std::fill(s->wv, s->wv + P, 0.0f); s->wt = 0; }
        std::vector<double> dl(P), hh(P); double l0 = 0;
        or_mlp_fd_eval(mp, s->p, s->z, tgt, c->fd_h, idx.data(), c->mlp_batch, dl.data(), hh.data(), &l0);
        or_fd_grad(P, dl.data(), hh.data(), grad.data());
        loss = l0;
    } else {
        std::vector<double> dl(c->mlp_pairs), ls(c->mlp_pairs);
        or_mlp_es_eval(mp, s->p, s->z, tgt, c->seed, it, c->mlp_sigma, c->mlp_pairs, idx.data(), c->mlp_batch, dl.data(), ls.data(), nullptr, nullptr);
        or_mlp_es_grad(P, c->mlp_pairs, c->seed, it, c->mlp_sigma, dl.data(), grad.data());
        double lmean = 0; for (int i = 0; i < c->mlp_pairs; i++) lmean += ls[i];
        loss = lmean / c->mlp_pairs;
    }
    s->wt++;
    or_adam(s->p, grad.data(), s->wm, s->wv, P, c->mlp_lr, s->wt);
    unsigned mask = 0;
    for (int l = 0; l < m.nlev; l++) if (!(c->qat > 0 && l == 0)) mask |= 1u << l;
    if (mask) {
        std::vector<float> zg(nz);
        or_lat_grad(mp, s->p, s->z, s->z, tgt, c->seed, s->lat_step_no, c->lat_sigma, c->lat_pairs, mask, nullptr, 0.0f, zg.data(), nullptr, nullptr, nullptr);
        s->zt++;
        or_adam(s->z, zg.data(), s->zm, s->zv, nz, c->lat_lr, s->zt);
        s->lat_step_no++;
    }
    if (c->qat > 0) {
        float grid[9 * 257]; or_qat_grid(grid);
        or_qat_search(mp, s->p, s->z, tgt, c->qat_ch, grid);
    }
    return loss;
}

}   // extern "C"

// mse_of, main.cpp:1764-1788: both images rounded to 8 bits as save_png does, squared differences per texture
extern "C" void or_mse_of(const float* a, const float* b, int W, int H, int nc, const float* w, float wsum, int ew, int eh,
                          double* tex, double* weighted) {
    const int T = nc / 3;
    if (ew <= 0 || ew > W) ew = W;
    if (eh <= 0 || eh > H) eh = H;
    double sse[4] = { 0, 0, 0, 0 };
    for (int yy = 0; yy < eh; yy++)
        for (int xx = 0; xx < ew; xx++) {
            const size_t p = (size_t)yy * W + xx;
            for (int t = 0; t < T; t++)
                for (int c = 0; c < 3; c++) {
                    const int xi = (int)std::lround(std::min(1.0f, std::max(0.0f, a[p * nc + 3 * t + c])) * 255.0f);
                    const int yi = (int)std::lround(std::min(1.0f, std::max(0.0f, b[p * nc + 3 * t + c])) * 255.0f);
                    const double d = (double)(xi - yi);
                    sse[t] += d * d;
                }
        }
    const double npix = (double)ew * eh;
    double ws = 0.0;
    for (int t = 0; t < T; t++) { tex[t] = sse[t] / (3.0 * npix); ws += (double)w[t] * sse[t]; }
    *weighted = ws / (3.0 * wsum * npix);
}


// ---------------------------------------------------------------- the progress print's statistics
namespace {
double cl0(double cnt, double tot) { return cnt != 0.0 && tot != 0.0 ? -std::log2(cnt / tot) : 0.0; }   // main.cpp:1130
// bits of channel c of level l as bitrate_stats charges it (main.cpp:2285-2288, 2297); *kind: 0 continuous, 1 discrete (qat), 2 --qes
int level_bits(const OrModel& m, const OrPrintIn& in, int l, int c, int* kind) {
    const bool fixed = l == 0 && in.qat > 0;
    const bool qes = in.qes_live && in.qes_bits[l] > 0;
    *kind = fixed ? 1 : (qes ? 2 : 0);
    if (fixed) return in.qat_ch[c];
    if (qes) return in.qes_bits[l];
    return (in.qes_on && in.qes_bits[l] > 0) ? in.qes_bits[l] : in.qbits;
}
// the quantization index of z[i] (channel c of level l) and its value
int level_index(const OrPrintIn& in, int kind, int l, int c, int bits, float lo, float range, float zi, float zdi, float* q) {
    const int levels = (1 << bits) - 1;
    if (kind == 1) { *q = zi; return qat_index(zi, bits); }
    if (kind == 2) { *q = zdi; return qes_index(zi, in.qes_lo[l * 64 + c], in.qes_range[l * 64 + c], levels); }
    const int k = or_q8_index(zi, lo, range, levels);
    *q = or_q8_value(k, lo, range, levels);
    return k;
}
int dpcm_pred(const int* idx, int W, int x, int y) {   // main.cpp:2336-2337
    const int lf = x ? idx[(size_t)y * W + x - 1] : -1, up = y ? idx[(size_t)(y - 1) * W + x] : -1;
    return (lf >= 0 && up >= 0) ? (lf + up) / 2 : (lf >= 0 ? lf : (up >= 0 ? up : 0));
}
}   // namespace

extern "C" {

// dct_analyze, main.cpp:1080-1208: the figures of the progress line (per-class bits, token counts, nz / lnz / eob-only)
void or_dct_analyze(const OrDct* d, int dc_raw_bits, int ctx, OrDctStats* out) {
    const int* zz = dct_tables().zigzag;
    OrDctStats S; memset(&S, 0, sizeof(S));
    const size_t nb = (size_t)d->BW * d->BH, nbc = nb * (size_t)d->C;
    S.nblk = (long long)nb;
    long long sum_nz = 0, sum_lnz = 0, n_lnz = 0, eob_only = 0;
    for (int c = 0; c < d->C; c++) {
        std::vector<size_t> run_cnt(65, 0), mag_cnt(257, 0), ctxr_cnt(64, 0), ctxm_cnt(64, 0);
        std::vector<size_t> ctx_run((size_t)64 * 65, 0), ctx_mag((size_t)64 * 257, 0), dcres_cnt(4097, 0);
        size_t nrun = 0, neob = 0;
        std::vector<int> dcs(nb, 0);
        for (size_t b = 0; b < nb; b++) {   // pass 1: counts
            const int16_t* sym = d->sym + (b * d->C + c) * 64;
            const int dc = sym[0];
            dcs[b] = dc;
            const int bx = (int)(b % d->BW), by = (int)(b / d->BW);
            const int pred = bx > 0 ? dcs[b - 1] : (by > 0 ? dcs[b - d->BW] : 0);
            dcres_cnt[(size_t)std::max(0, std::min(4096, dc - pred + 2048))]++;
            int run = 0, prev = 0, nz = 0, lnz = 0;
            for (int p = 1; p < 64; p++) {
                const int q = sym[zz[p]];
                if (q == 0) { run++; continue; }
                const int mag = std::min(256, std::abs(q)); if (std::abs(q) > 256) S.nmag_over++;
                run_cnt[run]++; mag_cnt[mag]++; ctx_run[(size_t)prev * 65 + run]++; ctx_mag[(size_t)prev * 257 + mag]++; ctxr_cnt[prev]++; ctxm_cnt[prev]++;
                nrun++; nz++; lnz = p; prev = p; run = 0;
            }
            if (lnz < 63) { run_cnt[64]++; ctx_run[(size_t)prev * 65 + 64]++; ctxr_cnt[prev]++; neob++; }
            sum_nz += nz;
            if (nz) { sum_lnz += lnz; n_lnz++; } else eob_only++;
        }
        S.ntok_nz += (long long)nrun; S.ntok_eob += (long long)neob;
        const size_t nruntok = nrun + neob;
        for (size_t b = 0; b < nb; b++) {   // pass 2: charge every token
            const int16_t* sym = d->sym + (b * d->C + c) * 64;
            const int bx = (int)(b % d->BW), by = (int)(b / d->BW);
            const int pred = bx > 0 ? dcs[b - 1] : (by > 0 ? dcs[b - d->BW] : 0);
            const double dcbits = cl0((double)dcres_cnt[(size_t)std::max(0, std::min(4096, sym[0] - pred + 2048))], (double)nb);
            S.raw[0] += dc_raw_bits; S.h0[0] += dcbits; S.ctx[0] += dcbits;
            int run = 0, prev = 0, lnz = 0;
            for (int p = 1; p < 64; p++) {
                const int q = sym[zz[p]];
                if (q == 0) { run++; continue; }
                const int mag = std::min(256, std::abs(q)); if (std::abs(q) > 256) S.nmag_over++;   // counted again, as main.cpp:1147 does
                const double r0 = cl0((double)run_cnt[run], (double)nruntok), m0 = cl0((double)mag_cnt[mag], (double)nrun);
                const double rc = cl0((double)ctx_run[(size_t)prev * 65 + run], (double)ctxr_cnt[prev]);
                const double mc = cl0((double)ctx_mag[(size_t)prev * 257 + mag], (double)ctxm_cnt[prev]);
                S.raw[1] += 7; S.raw[2] += 8; S.raw[3] += 1;
                S.h0[1] += r0; S.h0[2] += m0; S.h0[3] += 1;
                S.ctx[1] += rc; S.ctx[2] += mc; S.ctx[3] += 1;
                lnz = p; prev = p; run = 0;
            }
            if (lnz < 63) {
                S.raw[4] += 7; S.h0[4] += cl0((double)run_cnt[64], (double)nruntok); S.ctx[4] += cl0((double)ctx_run[(size_t)prev * 65 + 64], (double)ctxr_cnt[prev]);
            }
        }
        // scale codes: 4 bits raw, order-0, and the (up, left) context estimate of the BW x BH code grid (main.cpp:1162-1166,
        // context_entropy_bits main.cpp:2242-2258: H(X, U, L) - H(U, L), out-of-grid neighbours as code 0)
        size_t chist[16] = { 0 };
        for (size_t b = 0; b < nb; b++) chist[d->code[b * d->C + c]]++;
        double ch0 = 0; for (int k = 0; k < 16; k++) if (chist[k]) ch0 += (double)chist[k] * cl0((double)chist[k], (double)nb);
        double cctx = ch0;
        if (ctx) {
            std::vector<size_t> tri(4096, 0), pair(256, 0);
            for (int y = 0; y < d->BH; y++)
                for (int x = 0; x < d->BW; x++) {
                    const int s = d->code[((size_t)y * d->BW + x) * d->C + c];
                    const int u = y ? d->code[((size_t)(y - 1) * d->BW + x) * d->C + c] : 0;
                    const int l = x ? d->code[((size_t)y * d->BW + x - 1) * d->C + c] : 0;
                    tri[(size_t)u * 256 + l * 16 + s]++; pair[(size_t)u * 16 + l]++;
                }
            double hxul = 0, hul = 0;
            for (size_t i = 0; i < tri.size(); i++) if (tri[i]) hxul -= (double)tri[i] * std::log2((double)tri[i] / (double)nb);
            for (size_t i = 0; i < pair.size(); i++) if (pair[i]) hul -= (double)pair[i] * std::log2((double)pair[i] / (double)nb);
            cctx = hxul - hul;
        }
        S.code_raw += 4.0 * (double)nb; S.code_h0 += ch0; S.code_ctx += cctx;
        S.header += 3 * 32.0;
    }
    S.raw[5] = S.code_raw; S.h0[5] = S.code_h0; S.ctx[5] = S.code_ctx;
    S.raw[6] = S.h0[6] = S.ctx[6] = S.header;
    for (int k = 0; k < 7; k++) { S.raw_total += S.raw[k]; S.h0_total += S.h0[k]; S.ctx_total += S.ctx[k]; }
    S.nz_mean = nbc ? (double)sum_nz / (double)nbc : 0;
    S.lnz_mean = n_lnz ? (double)sum_lnz / (double)n_lnz : 0;
    S.eob_only_frac = nbc ? (double)eob_only / (double)nbc : 0;
    *out = S;
}

// bitrate_stats, main.cpp:2273-2352 as a progress print runs it (order-0 in place of the context estimate)
void or_bitrate_stats(const OrModel* mp, const OrPrintIn* in, long long P, const float* z, const float* zdec, OrBitrate* out, float* zq) {
    const OrModel& m = *mp;
    OrBitrate s; memset(&s, 0, sizeof(s));
    const double npix = (double)m.W * m.H;
    const long long nz = nzof(m);
    s.bits_mlp = (double)P * 16.0;
    s.bpp_fp32 = ((double)nz * 32.0 + (double)P * 32.0) / npix;
    double ent = 0, header = 0, raw = 0, ctxb = 0, est = 0;
    for (int l = 0; l < m.nlev; l++) {
        const OrLevel& L = m.lv[l];
        const size_t nl = (size_t)L.W * L.H * L.C;
        const double ntex = (double)L.W * L.H;
        float* q = zq + L.off;
        if (l == 0 && in->dct_live) {
            OrDctStats b; or_dct_analyze(in->dct, in->dc_raw_bits, 0, &b);
            raw += b.raw_total - b.header; ent += b.h0_total - b.header; ctxb += b.ctx_total - b.header; est += b.h0_total - b.header;
            s.bpp_ctx_level0 += (b.ctx_total - b.header) / npix;
            header += b.header;
            memcpy(q, zdec + L.off, nl * sizeof(float));
            continue;
        }
        int kind0; (void)level_bits(m, *in, l, 0, &kind0);
        if (kind0 == 0) raw += (double)nl * (double)level_bits(m, *in, l, 0, &kind0);
        for (int c = 0; c < L.C; c++) {
            int kind; const int bits = level_bits(m, *in, l, c, &kind);
            const int levels = (1 << bits) - 1;
            if (kind != 0) raw += ntex * (double)bits;
            float lo = 1e30f, hi = -1e30f;
            if (kind == 0) for (size_t i = c; i < nl; i += L.C) { lo = std::min(lo, z[L.off + i]); hi = std::max(hi, z[L.off + i]); }
            const float range = std::max(hi - lo, 1e-6f);
            std::vector<int> hist(levels + 1, 0), idx((size_t)L.W * L.H);
            for (size_t i = c, t = 0; i < nl; i += L.C, t++) {
                const int qi = level_index(*in, kind, l, c, bits, lo, range, z[L.off + i], zdec[L.off + i], &q[i]);
                hist[qi]++; idx[t] = qi;
            }
            double h0 = 0;
            for (int v = 0; v <= levels; v++) if (hist[v]) h0 -= hist[v] * std::log2(hist[v] / ntex);
            ent += h0;
            if (l == 0) { ctxb += h0; s.bpp_ctx_level0 += h0 / npix; est += h0; }
            else {
                ctxb += h0;
                std::vector<int> rh(levels + 1, 0);
                for (int y = 0; y < L.H; y++)
                    for (int x = 0; x < L.W; x++) rh[(idx[(size_t)y * L.W + x] - dpcm_pred(idx.data(), L.W, x, y)) & levels]++;
                double hr = 0;
                for (int v = 0; v <= levels; v++) if (rh[v]) hr -= rh[v] * std::log2(rh[v] / ntex);
                est += hr;
            }
        }
        if (kind0 != 1) header += L.C * 2 * 32.0;
    }
    s.bpp_q8 = (raw + header + s.bits_mlp) / npix;
    s.bpp_q8_ent = (ent + header + s.bits_mlp) / npix;
    s.bpp_q8_ctx = (ctxb + header + s.bits_mlp) / npix;
    s.bpp_est = (est + header + s.bits_mlp) / npix;
    s.bits_raw_latent = raw; s.bits_header = header;
    *out = s;
}

// latent_stats, main.cpp:2211-2216
void or_latent_stats(const OrModel* m, int l, const float* z, float* mean, float* sd, float* mx) {
    const OrLevel& L = m->lv[l];
    const size_t n = (size_t)L.W * L.H * L.C;
    double s = 0, s2 = 0; float x = 0;
    for (size_t i = 0; i < n; i++) { const float v = z[L.off + i]; s += v; s2 += (double)v * v; x = std::max(x, std::fabs(v)); }
    *mean = (float)(s / n);
    *sd = (float)std::sqrt(std::max(0.0, s2 / n - (s / n) * (s / n)));
    *mx = x;
}

void or_print_counts_size(const OrModel* mp, const OrPrintIn* in, long long* n_bitrate, long long* n_dct) {
    long long nb = 0;
    for (int l = 0; l < mp->nlev; l++) {
        if (l == 0 && in->dct_live) continue;
        for (int c = 0; c < mp->lv[l].C; c++) { int kind; nb += (long long)(1 << level_bits(*mp, *in, l, c, &kind)) * (l >= 1 ? 2 : 1); }
    }
    *n_bitrate = nb;
    *n_dct = in->dct_live ? (long long)in->dct->C * OR_DCT_COUNTS_PER_CH + OR_DCT_COUNTS_TAIL : 0;
}

void or_print_counts(const OrModel* mp, const OrPrintIn* in, const float* z, const float* zdec, long long* bitrate, float* lohi,
                     long long* dct) {
    const OrModel& m = *mp;
    long long nb_, nd_; or_print_counts_size(mp, in, &nb_, &nd_);
    memset(bitrate, 0, (size_t)nb_ * sizeof(long long));
    long long* h = bitrate;
    for (int l = 0; l < m.nlev; l++) {
        const OrLevel& L = m.lv[l];
        if (l == 0 && in->dct_live) continue;
        const size_t nl = (size_t)L.W * L.H * L.C;
        for (int c = 0; c < L.C; c++) {
            int kind; const int bits = level_bits(m, *in, l, c, &kind);
            const int nbin = 1 << bits;
            float lo = 1e30f, hi = -1e30f;
            if (kind == 0) for (size_t i = c; i < nl; i += L.C) { lo = std::min(lo, z[L.off + i]); hi = std::max(hi, z[L.off + i]); }
            lohi[(l * 64 + c) * 2] = lo; lohi[(l * 64 + c) * 2 + 1] = hi;
            const float range = std::max(hi - lo, 1e-6f);
            std::vector<int> idx((size_t)L.W * L.H);
            for (size_t i = c, t = 0; i < nl; i += L.C, t++) { float q; idx[t] = level_index(*in, kind, l, c, bits, lo, range, z[L.off + i], zdec[L.off + i], &q); h[idx[t]]++; }
            h += nbin;
            if (l >= 1) {
                for (int y = 0; y < L.H; y++)
                    for (int x = 0; x < L.W; x++) h[(idx[(size_t)y * L.W + x] - dpcm_pred(idx.data(), L.W, x, y)) & (nbin - 1)]++;
                h += nbin;
            }
        }
    }
    if (!in->dct_live) return;
    const OrDct* d = in->dct;
    const int* zz = dct_tables().zigzag;
    memset(dct, 0, (size_t)nd_ * sizeof(long long));
    const size_t nb = (size_t)d->BW * d->BH;
    long long* tail = dct + (size_t)d->C * OR_DCT_COUNTS_PER_CH;
    for (int c = 0; c < d->C; c++) {
        long long* runh = dct + (size_t)c * OR_DCT_COUNTS_PER_CH;
        long long *mag = runh + 65, *cr = mag + 257, *cm = cr + 64 * 65, *ctxr = cm + 64 * 257, *ctxm = ctxr + 64, *dcres = ctxm + 64;
        long long *code = dcres + 4097, *tri = code + 16, *pair = tri + 4096, *sc = pair + 256;   // sc: nrun neob nsign
        for (size_t b = 0; b < nb; b++) {
            const int16_t* sym = d->sym + (b * d->C + c) * 64;
            const int bx = (int)(b % d->BW), by = (int)(b / d->BW);
            const int pred = bx > 0 ? d->sym[((b - 1) * d->C + c) * 64] : (by > 0 ? d->sym[((b - d->BW) * d->C + c) * 64] : 0);
            dcres[std::max(0, std::min(4096, sym[0] - pred + 2048))]++;
            int run = 0, prev = 0, nz = 0, lnz = 0;
            for (int p = 1; p < 64; p++) {
                const int q = sym[zz[p]];
                if (q == 0) { run++; continue; }
                const int mg = std::min(256, std::abs(q)); if (std::abs(q) > 256) tail[4]++;
                runh[run]++; mag[mg]++; cr[prev * 65 + run]++; cm[prev * 257 + mg]++; ctxr[prev]++; ctxm[prev]++;
                sc[0]++; sc[2]++; nz++; lnz = p; prev = p; run = 0;
            }
            if (lnz < 63) { runh[64]++; cr[prev * 65 + 64]++; ctxr[prev]++; sc[1]++; }
            tail[0] += nz;
            if (nz) { tail[1] += lnz; tail[2]++; } else tail[3]++;
            const int k = d->code[b * d->C + c];
            code[k]++;
            const int u = by ? d->code[(b - d->BW) * d->C + c] : 0, lf = bx ? d->code[(b - 1) * d->C + c] : 0;
            tri[u * 256 + lf * 16 + k]++; pair[u * 16 + lf]++;
        }
    }
}

int or_host_isa_level(void) {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("avx512cd") &&
        __builtin_cpu_supports("avx512dq") && __builtin_cpu_supports("avx512vl"))
        return 4;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("bmi2")) return 3;
    return 1;
}

}   // extern "C"
