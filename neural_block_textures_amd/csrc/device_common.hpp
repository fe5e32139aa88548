// Device-side building blocks of the gfx950 ES backend: the model description every kernel
// receives by value, the counter-based noise, the sampling geometry and the MLP evaluator.
//
// Floating point: every .hip file is compiled with -ffp-contract=off; a fused multiply-add
// appears only where it is written as __builtin_fmaf, at exactly the places where the
// reference's host build fuses (the oracle writes the same fmaf calls). Division and sqrt are
// IEEE-rounded (hipcc's default). The one function with a different last bit in rare cases is
// expf in the sigmoid output (the device's expf against the host C library's).
#pragma once
#ifdef __HIPCC_RTC__   // hipRTC provides the runtime itself and the fixed-width integer types in its own namespace
using __hip_internal::int8_t; using __hip_internal::int16_t; using __hip_internal::int32_t; using __hip_internal::int64_t;
using __hip_internal::uint8_t; using __hip_internal::uint16_t; using __hip_internal::uint32_t; using __hip_internal::uint64_t;
#else
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

#include "noise_math.hpp"

namespace ntc_hip {

constexpr int kMaxLevels = 3, kMaxPos = 16, kMaxOut = 12, kMaxHidden = 8, kMaxWidth = 64;
// The minibatch arrays of a trainer (structure of arrays, Mcap slots per row): the feature array has
// minibatch_rows(nin) rows, those past nin zero (the matrix kernels read whole 4-input k-steps), and both
// arrays carry kMinibatchSlack floats past their last row (more than the 7 tile strides of 32 slots a
// population pass can read past the end of its chunk).
constexpr int kMinibatchSlack = 256;
__host__ __device__ constexpr int minibatch_rows(int nin) { return 4 * ((nin + 3) / 4); }

// ---------------------------------------------------------------- model description
struct DevLevel {
    int W, H, C, nearest;
    long long off;       // first value of the level in the flat latent vector
    int rng;             // offset of the level's footprint ranges in the range table: xb[W] xe[W] yb[H] ye[H]
    int pad;
};

struct DevModel {
    int W, H, npix, nout;
    int nin, nlev, npos, nl;
    DevLevel lv[kMaxLevels];
    int pos[kMaxPos];
    int hidden[kMaxHidden];
    float leak;
    int clamp_out;
    float cw[kMaxOut];
    float wsum;
    float inv_px;        // 1 / (3 wsum W H), float, as LatentTrainer computes it
    int P;               // MLP parameter count
    float fold_c;        // (1 - leak) / (1 + leak): the folded activation's constant, divided once on the host
    long long nz;        // latent floats
};


// ---------------------------------------------------------------- counter-based noise
// The key and Box-Muller draw of the reference's cuda/ntc_noise.h:20-47: a splitmix64 output
// function over (seed, stream, step, pair) for the stream head, then over head + index * phi64.
enum : uint32_t { NS_LAT = 1, NS_MLP = 2, NS_BATCH_PIX = 3, NS_BATCH_TEX = 4 };
constexpr uint64_t kPhi64 = 0x9E3779B97F4A7C15ull;

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t x) {
    x += kPhi64;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
__host__ __device__ __forceinline__ uint64_t noise_head(uint64_t seed, uint32_t stream, uint32_t step, uint32_t pair) {
    return mix64(seed ^ ((uint64_t)stream << 56) ^ ((uint64_t)step << 32) ^ (uint64_t)pair);
}
__host__ __device__ __forceinline__ uint64_t noise_bits(uint64_t head, uint64_t index) { return mix64(head + index * kPhi64); }
// x is not a NaN, decided on its bits (valid in code compiled to assume no NaNs, where a float test folds away)
__device__ __forceinline__ bool not_nan_bits(float x) { return (__float_as_uint(x) & 0x7fffffffu) <= 0x7f800000u; }
__host__ __device__ __forceinline__ uint32_t noise_uniform(uint32_t u, uint32_t n) { return (uint32_t)(((uint64_t)u * (uint64_t)n) >> 32); }
// One standard normal draw: the 24-bit halves of the key select the two factors, whose product
// is the reference's sqrtf(-2 logf(u1)) * cosf(2 pi u2) bit for bit (one IEEE multiply).
__device__ __forceinline__ float gauss_at(const NoiseFix& fx, uint64_t head, uint64_t index) {
    const uint64_t h = noise_bits(head, index);
    return __fmul_rn(nm_radius(fx, (uint32_t)(h >> 40)), nm_cosine(fx, (uint32_t)(h & 0xFFFFFFull)));
}

// ---------------------------------------------------------------- geometry (main.cpp:507-547)
struct Tap { int x0, x1, y0, y1; float fx, fy; };

__host__ __device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// bilinear_tap (main.cpp:512-531); the bilinear coordinate is a rounded product then a rounded
// difference, as the reference's build evaluates it
__host__ __device__ __forceinline__ Tap tap_of(int LW, int LH, bool nearest, float u, float v) {
    Tap t;
    if (nearest) {
        const float x = u * (float)LW, y = v * (float)LH;
        const int ix = (int)floorf(x), iy = (int)floorf(y);
        t.fx = x - (float)ix; t.fy = y - (float)iy;
        t.x0 = t.x1 = clampi(ix, 0, LW - 1);
        t.y0 = t.y1 = clampi(iy, 0, LH - 1);
        return t;
    }
    const float x = u * (float)LW - 0.5f, y = v * (float)LH - 0.5f;
    const int x0 = (int)floorf(x), y0 = (int)floorf(y);
    t.fx = x - (float)x0; t.fy = y - (float)y0;
    t.x0 = clampi(x0, 0, LW - 1); t.x1 = clampi(x0 + 1, 0, LW - 1);
    t.y0 = clampi(y0, 0, LH - 1); t.y1 = clampi(y0 + 1, 0, LH - 1);
    return t;
}
__host__ __device__ __forceinline__ float pixel_u(int px, int W) { return ((float)px + 0.5f) / (float)W; }

struct Blend { float w00, w10, w01, w11; };
__device__ __forceinline__ Blend blend_of(const Tap& t) {
    Blend b;
    b.w00 = (1.0f - t.fx) * (1.0f - t.fy); b.w10 = t.fx * (1.0f - t.fy);
    b.w01 = (1.0f - t.fx) * t.fy;          b.w11 = t.fx * t.fy;
    return b;
}
// main.cpp:546 as the reference's build fuses it: w11 d + (w01 c + (w00 a + w10 b))
__device__ __forceinline__ float blend(const Blend& b, float a, float bb, float c, float d) {
    return __builtin_fmaf(b.w11, d, __builtin_fmaf(b.w01, c, __builtin_fmaf(b.w00, a, __fmul_rn(b.w10, bb))));
}

// Texel sources for the feature builder: the plain decode buffer, or the decode buffer with the
// latent-ES perturbation of one antithetic member applied texel by texel
// (zp = zb + sg * eps as one fused operation, main.cpp:1999-2000).
struct PlainLatent {
    const float* z;
    __device__ __forceinline__ float operator()(int /*l*/, long long i) const { return z[i]; }
};
struct PerturbedLatent {
    const float* z; const float* eps; float sg; unsigned mask;
    __device__ __forceinline__ float operator()(int l, long long i) const {
        return ((mask >> l) & 1u) ? __builtin_fmaf(sg, eps[i], z[i]) : z[i];
    }
};

// sample_latent (main.cpp:533-547) of channels [0, C) of level l into f
template <int CMAX, class Src>
__device__ __forceinline__ void sample_level(const DevLevel& L, int l, const Src& src, const Tap& t, int C, float* f) {
    const long long a = L.off + ((long long)t.y0 * L.W + t.x0) * L.C;
    if (L.nearest) {
#pragma unroll
        for (int c = 0; c < CMAX; c++) if (c < C) f[c] = src(l, a + c);
        return;
    }
    const long long b = L.off + ((long long)t.y0 * L.W + t.x1) * L.C;
    const long long cc = L.off + ((long long)t.y1 * L.W + t.x0) * L.C;
    const long long d = L.off + ((long long)t.y1 * L.W + t.x1) * L.C;
    const Blend w = blend_of(t);
#pragma unroll
    for (int c = 0; c < CMAX; c++) if (c < C) f[c] = blend(w, src(l, a + c), src(l, b + c), src(l, cc + c), src(l, d + c));
}

// ---------------------------------------------------------------- MLP shapes
// A compile-time shape: level channel counts, positional generators, uniform hidden width and
// depth, outputs. Everything is unrolled; weight addresses are uniform per wave, so the
// weights stream through the scalar cache into SGPRs and every MAC is one v_fma_f32.
template <int C0_, int C1_, int C2_, int NPOS_, int H_, int NL_, int NOUT_>
struct FixedShape {
    static constexpr bool kFixed = true, kUniform = true;
    static constexpr int kC0 = C0_, kC1 = C1_, kC2 = C2_, kNpos = NPOS_, kH = H_, kNL = NL_, kNout = NOUT_;
    static constexpr int kNin = C0_ + C1_ + C2_ + 2 * NPOS_;
    static constexpr int kMaxIn = kNin, kMaxOut = NOUT_, kMaxH = H_;
    static constexpr int kLevels = C2_ > 0 ? 3 : (C1_ > 0 ? 2 : 1);
    static constexpr int width(int) { return H_; }   // units of hidden layer l
    static bool matches(const DevModel& m) {
        if (m.nlev != kLevels || m.npos != kNpos || m.nl != kNL || m.nout != kNout || m.nin != kNin) return false;
        const int c[3] = { kC0, kC1, kC2 };
        for (int l = 0; l < m.nlev; l++) if (m.lv[l].C != c[l]) return false;
        for (int l = 0; l < m.nl; l++) if (m.hidden[l] != kH) return false;
        return true;
    }
};
// The same with a width per hidden layer (H_...: layer 0 first), for the VALU kernels only (the matrix
// kernels tile one width): the kernels compiled at init for a model whose hidden layers differ in width.
template <int C0_, int C1_, int C2_, int NPOS_, int NOUT_, int... H_>
struct FixedShapeW {
    static constexpr bool kFixed = true, kUniform = false;
    static constexpr int kC0 = C0_, kC1 = C1_, kC2 = C2_, kNpos = NPOS_, kNL = (int)sizeof...(H_), kNout = NOUT_;
    static constexpr int kNin = C0_ + C1_ + C2_ + 2 * NPOS_;
    static constexpr int kW[sizeof...(H_)] = { H_... };
    static constexpr int width(int l) { return kW[l]; }
    static constexpr int max_width() {
        int w = 0;
        for (int l = 0; l < kNL; l++) w = kW[l] > w ? kW[l] : w;
        return w;
    }
    static constexpr int kMaxIn = kNin, kMaxOut = NOUT_, kMaxH = max_width();
    static constexpr int kLevels = C2_ > 0 ? 3 : (C1_ > 0 ? 2 : 1);
    static bool matches(const DevModel& m) {
        if (m.nlev != kLevels || m.npos != kNpos || m.nl != kNL || m.nout != kNout || m.nin != kNin) return false;
        const int c[3] = { kC0, kC1, kC2 };
        for (int l = 0; l < m.nlev; l++) if (m.lv[l].C != c[l]) return false;
        for (int l = 0; l < m.nl; l++) if (m.hidden[l] != kW[l]) return false;
        return true;
    }
};
// Any shape inside the envelope: runtime loops over per-thread arrays.
struct RuntimeShape {
    static constexpr bool kFixed = false, kUniform = false;
    static constexpr int kC0 = 16, kC1 = 64, kC2 = 64, kNpos = kMaxPos;
    static constexpr int kMaxIn = kMaxWidth, kMaxOut = ntc_hip::kMaxOut;
    static bool matches(const DevModel&) { return true; }
};

// Decoder::features + PosEnc::encode (main.cpp:1593-1608, 1687-1702) into f[0, nin)
template <class S, class Src>
__device__ __forceinline__ void features(const DevModel& m, const Src& src, int px, int py, float (&f)[S::kMaxIn]) {
    const float u = pixel_u(px, m.W), v = pixel_u(py, m.H);
    const Tap t0 = tap_of(m.lv[0].W, m.lv[0].H, m.lv[0].nearest != 0, u, v);
    Tap t1 = t0;
    if constexpr (S::kFixed) {
        sample_level<S::kC0>(m.lv[0], 0, src, t0, S::kC0, f);
        if constexpr (S::kC1 > 0) {
            t1 = tap_of(m.lv[1].W, m.lv[1].H, m.lv[1].nearest != 0, u, v);
            sample_level<S::kC1>(m.lv[1], 1, src, t1, S::kC1, f + S::kC0);
        }
        if constexpr (S::kC2 > 0) {
            const Tap t2 = tap_of(m.lv[2].W, m.lv[2].H, m.lv[2].nearest != 0, u, v);
            sample_level<S::kC2>(m.lv[2], 2, src, t2, S::kC2, f + S::kC0 + S::kC1);
        }
        constexpr int k0 = S::kC0 + S::kC1 + S::kC2;
#pragma unroll
        for (int q = 0; q < S::kNpos; q++) {
            const bool uv = m.pos[q] == 0;
            f[k0 + 2 * q] = __builtin_fmaf(uv ? u : t1.fx, 2.0f, -1.0f);
            f[k0 + 2 * q + 1] = __builtin_fmaf(uv ? v : t1.fy, 2.0f, -1.0f);
        }
    } else {
        int k = 0;
        for (int l = 0; l < m.nlev; l++) {
            const Tap tl = l == 0 ? t0 : tap_of(m.lv[l].W, m.lv[l].H, m.lv[l].nearest != 0, u, v);
            if (l == 1) t1 = tl;
            float tmp[kMaxWidth];
            sample_level<kMaxWidth>(m.lv[l], l, src, tl, m.lv[l].C, tmp);
            for (int c = 0; c < m.lv[l].C; c++) f[k + c] = tmp[c];
            k += m.lv[l].C;
        }
        for (int q = 0; q < m.npos; q++) {
            const bool uv = m.pos[q] == 0;
            f[k++] = __builtin_fmaf(uv ? u : t1.fx, 2.0f, -1.0f);
            f[k++] = __builtin_fmaf(uv ? v : t1.fy, 2.0f, -1.0f);
        }
    }
}

// a read-only view of global memory; uniform addresses in it become scalar loads
typedef __attribute__((address_space(4))) float CFloat;

// Thread and workgroup ids read straight from the hardware. Kernels built with IEEE mode off cannot inline
// the device library's id helpers (built with it on): blockIdx / threadIdx then become calls that return
// VGPRs, every block-uniform index derived from them is treated as divergent (VALU address arithmetic,
// divergent branches, waterfall loops over buffer descriptors). The builtins keep workgroup ids in SGPRs.
__device__ __forceinline__ int tid_x() { return (int)__builtin_amdgcn_workitem_id_x(); }
__device__ __forceinline__ int bid_x() { return (int)__builtin_amdgcn_workgroup_id_x(); }
__device__ __forceinline__ int bid_y() { return (int)__builtin_amdgcn_workgroup_id_y(); }

// A raw buffer over `bytes` bytes at p: a load takes a 32-bit byte offset per lane (VGPR) and one per wave
// (SGPR), and one past the end returns 0 instead of faulting.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const float* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float buffer_f32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}

// A pointer every lane holds the same value of, moved to SGPRs (a value that flowed through a
// loop with a per-lane trip count is otherwise treated as divergent).
__device__ __forceinline__ const float* uniform_ptr(const float* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return (const float*)(((uint64_t)hi << 32) | lo);
}

// Adam::step (main.cpp:1793-1810) on parameter i given its gradient; c1, c2 from the host's powf
__device__ __forceinline__ void adam_at(float* __restrict__ theta, float* __restrict__ m, float* __restrict__ v, size_t i, float gi,
                                        float lr, float c1, float c2) {
    const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    const float ob1 = 1.0f - b1, ob2 = 1.0f - b2;
    const float mi = __builtin_fmaf(b1, m[i], __fmul_rn(ob1, gi));
    const float vi = __builtin_fmaf(b2, v[i], __fmul_rn(__fmul_rn(ob2, gi), gi));
    m[i] = mi; v[i] = vi;
    const float mh = mi / c1, vh = vi / c2;
    theta[i] = theta[i] - (lr * mh) / (__builtin_sqrtf(vh) + eps);
}

// Adam on values already loaded (the same operations as adam_at)
__device__ __forceinline__ void adam_vals(float& theta, float& m, float& v, float gi, float lr, float c1, float c2) {
    const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    const float ob1 = 1.0f - b1, ob2 = 1.0f - b2;
    m = __builtin_fmaf(b1, m, __fmul_rn(ob1, gi));
    v = __builtin_fmaf(b2, v, __fmul_rn(__fmul_rn(ob2, gi), gi));
    const float mh = m / c1, vh = v / c2;
    theta = theta - (lr * mh) / (__builtin_sqrtf(vh) + eps);
}

__device__ __forceinline__ float activate(float x, float leak) { return x > 0.0f ? x : leak * x; }   // main.cpp:560
__device__ __forceinline__ float output_of(float s, int clamp_out) {                                  // main.cpp:624-625
    return clamp_out ? fminf(1.0f, fmaxf(0.0f, s + 0.5f)) : 1.0f / (1.0f + expf(-s));
}

// mlp_forward (main.cpp:603-627): per unit s = b[j], then s = fma(w[j][i], a[i], s) for i
// ascending; w is the flat parameter vector (per layer W[out][in] row-major, then b[out]).
// Hidden layers L .. kNL - 1 of a fixed shape, one compile-time layer at a time (every width a constant,
// so the activations stay in registers): a holds layer L - 1's outputs, p points at layer L's weights.
template <class S, int L>
__device__ __forceinline__ void mlp_hidden_from(const DevModel& m, const CFloat*& p, float (&a)[S::kMaxH]) {
    if constexpr (L < S::kNL) {
        constexpr int HI = S::width(L - 1), HO = S::width(L);
        float t[HO];
        const CFloat* b = p + HO * HI;
#pragma unroll
        for (int j = 0; j < HO; j++) {
            float s = b[j];
#pragma unroll
            for (int i = 0; i < HI; i++) s = __builtin_fmaf(p[j * HI + i], a[i], s);
            t[j] = activate(s, m.leak);
        }
#pragma unroll
        for (int j = 0; j < HO; j++) a[j] = t[j];
        p = b + HO;
        mlp_hidden_from<S, L + 1>(m, p, a);
    }
}

template <class S>
__device__ __forceinline__ void mlp_forward(const DevModel& m, const float* __restrict__ w, const float (&in)[S::kMaxIn],
                                            float (&out)[S::kMaxOut]) {
    if constexpr (S::kFixed) {
        constexpr int NIN = S::kNin, H0 = S::width(0), HL = S::width(S::kNL - 1), NO = S::kNout;
        // The weights are read through the constant address space from an SGPR address, so every
        // load is a scalar load into SGPRs; laundering the address through an empty asm keeps the
        // loads inside the caller's pixel loop (hoisted, the P loop-invariant weights overflow the
        // SGPRs and every FMA pays a v_readlane).
        w = uniform_ptr(w);
        asm volatile("" : "+s"(w));
        const CFloat* __restrict__ wc = (const CFloat*)w;
        float a[S::kMaxH];
        {
            const CFloat* b = wc + H0 * NIN;
#pragma unroll
            for (int j = 0; j < H0; j++) {
                float s = b[j];
#pragma unroll
                for (int i = 0; i < NIN; i++) s = __builtin_fmaf(wc[j * NIN + i], in[i], s);
                a[j] = activate(s, m.leak);
            }
        }
        const CFloat* p = wc + H0 * NIN + H0;
        mlp_hidden_from<S, 1>(m, p, a);
        const CFloat* b = p + NO * HL;
#pragma unroll
        for (int j = 0; j < NO; j++) {
            float s = b[j];
#pragma unroll
            for (int i = 0; i < HL; i++) s = __builtin_fmaf(p[j * HL + i], a[i], s);
            out[j] = output_of(s, m.clamp_out);
        }
    } else {
        float bufA[kMaxWidth], bufB[kMaxWidth];
        for (int i = 0; i < m.nin; i++) bufA[i] = in[i];
        float* cur = bufA; float* nxt = bufB;
        int ncur = m.nin;
        const float* p = w;
        for (int l = 0; l < m.nl; l++) {
            const int nh = m.hidden[l];
            const float* b = p + nh * ncur;
            for (int j = 0; j < nh; j++) {
                float s = b[j];
                for (int i = 0; i < ncur; i++) s = __builtin_fmaf(p[j * ncur + i], cur[i], s);
                nxt[j] = activate(s, m.leak);
            }
            p = b + nh; ncur = nh;
            float* tmp = cur; cur = nxt; nxt = tmp;
        }
        const float* b = p + m.nout * ncur;
        for (int j = 0; j < m.nout; j++) {
            float s = b[j];
            for (int i = 0; i < ncur; i++) s = __builtin_fmaf(p[j * ncur + i], cur[i], s);
            out[j] = output_of(s, m.clamp_out);
        }
    }
}

// Per-pixel weighted squared error: float products summed into a double (loss_subset,
// main.cpp:1747) or fused into a float (decode_err, main.cpp:1731-1732).
template <int NOMAX>
__device__ __forceinline__ double pixel_err_d(const DevModel& m, const float (&o)[NOMAX], const float* t) {
    double s = 0.0;
#pragma unroll
    for (int c = 0; c < NOMAX; c++) if (c < m.nout) { const float d = o[c] - t[c]; s += (double)__fmul_rn(m.cw[c], __fmul_rn(d, d)); }
    return s;
}
template <int NOMAX>
__device__ __forceinline__ float pixel_err_f(const DevModel& m, const float (&o)[NOMAX], const float* t) {
    float e = 0.0f;
#pragma unroll
    for (int c = 0; c < NOMAX; c++) if (c < m.nout) { const float d = o[c] - t[c]; e = __builtin_fmaf(m.cw[c], __fmul_rn(d, d), e); }
    return e;
}

// qes_index (main.cpp:448-453): the --qes grid index, round half to even, clamped in float before the cast
__device__ __forceinline__ int qes_index(float v, float lo, float range, int levels) {
    const float r = rintf(((v - lo) / range) * (float)levels);   // round half to even
    if (!(r == r)) return 0;
    return r <= 0.0f ? 0 : (r >= (float)levels ? levels : (int)r);
}
// q8_index / q8_value (main.cpp:478-482): the post-hoc grid of a continuous level, strict float
__device__ __forceinline__ int q8_index(float z, float lo, float range, int levels) {
    const float x = __fmul_rn(__fdiv_rn(__fsub_rn(z, lo), range), (float)levels);
    const float r = roundf(x);                                   // lround: half away from zero
    return r <= 0.0f ? 0 : (r >= (float)levels ? levels : (int)r);
}
__device__ __forceinline__ float q8_value(int k, float lo, float range, int levels) {
    return __fadd_rn(lo, __fmul_rn(__fdiv_rn((float)k, (float)levels), range));
}

// qat_index (main.cpp:2060-2064): lround of the grid coordinate, clamped
__device__ __forceinline__ int qat_index(float v, int bits) {
    const int levels = (1 << bits) - 1;
    const int k = (int)roundf((v + 1.0f) * 0.5f * (float)levels);
    return clampi(k, 0, levels);
}

// ---------------------------------------------------------------- reductions (wave64)
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
// Fixed-order block sum of doubles for blockDim.x = BLOCK: butterfly within each wave, then the
// wave sums in wave order. The result is valid in every thread.
template <int BLOCK>
__device__ __forceinline__ double block_sum(double v, double* lds /* BLOCK / 64 */) {
    v = wave_sum(v);
    const int lane = tid_x() & 63, wid = tid_x() >> 6;
    if (lane == 0) lds[wid] = v;
    __syncthreads();
    double r = 0.0;
#pragma unroll
    for (int i = 0; i < BLOCK / 64; i++) r += lds[i];
    __syncthreads();
    return r;
}

}   // namespace ntc_hip
