// The MLP of the fixed shapes on the FP32 matrix cores of gfx950 (v_mfma_f32_16x16x4f32).
//
// One wave evaluates one member's MLP on a tile of 16 pixels at a time, with the member's
// parameters held in VGPRs in the instruction's operand layout:
//   A (16 x 4)  lane l holds A[l % 16][l / 16]        weights W[out][in]: out = 16 ot + l % 16
//   B (4 x 16)  lane l holds B[l / 16][l % 16]        activations: unit 4 ks + l / 16 of pixel l % 16
//   C/D (16x16) lane l, register r holds D[4 (l / 16) + r][l % 16]
// On gfx950 this instruction computes D = C then D = fma(A[.][k], B[k][.], D) for k = 0..3 in
// order, each step rounded (measured against host fmaf chains on 1 M random values, including
// subnormal operands, with no difference). With C = the bias and the k-steps of a layer taken in
// ascending input order, every unit is therefore the reference's s = b[j]; s = fma(w[j][i], a[i], s)
// for i ascending (main.cpp:603-627), bit for bit.
//
// A layer's output comes back in the D layout (lane group g holds units 4g + r of a 16-unit
// tile); the next layer wants lane group q to hold unit 4 ks + q. A 4 x 4 transpose across
// (lane group, register) - two v_permlane32_swap and two v_permlane16_swap per 16-unit tile -
// turns the activated D registers of tile t into the B operands of k-steps 4t .. 4t + 3.
//
// Hidden widths that are not a multiple of 16 pad the last tile with zero weights and biases. Its
// rows are ordered so that the units sit in the first registers of the four lane groups (row 4g + r
// holds unit 4r + g of the tile): the registers past the last unit hold padding only, and the next
// layer skips their k-steps (36 units: 9 k-steps, not 12). Padded rows compute fma(0, x, 0) chains
// and activate to zero, so the real units are unchanged.
#pragma once
#include "device_common.hpp"

namespace ntc_hip {

typedef float f4v __attribute__((ext_vector_type(4)));

// The least fraction of model multiply-adds in a shape's matrix instructions for the matrix cores to
// take it. A 16x16x4 instruction does 32 multiply-adds per cycle, a VALU FMA 16, so 0.5 breaks even
// on the multiply-adds alone; the matrix kernels also spend fewer VALU instructions per tile on
// everything else, and on the MI355X 17-wide hidden layers (42-47%) ran 5-11% faster per ES
// iteration on them (and their central-difference populations, with the exact two-instruction leaky
// activation, 9-10% faster per launch); 7-wide ones (38%) are left to the VALU.
#ifndef NTC_MFMA_MIN_USEFUL
#define NTC_MFMA_MIN_USEFUL 0.4
#endif

// The fraction of the multiply-adds of a 16-pixel tile's matrix instructions that are the model's, for
// an nin -> H (x NL hidden layers) -> nout MLP with the hidden tiles padded to 16 units and the padding's
// k-steps skipped, and whether that pays off (NTC_MFMA_MIN_USEFUL).
// (models with at most 4 outputs take their output layer on the VALU in either case: only their hidden
// layers count)
__host__ __device__ constexpr int mfma_per_tile(int nin, int H, int NL, int nout) {
    return ((H + 15) / 16) * ((nin + 3) / 4) + (NL - 1) * ((H + 15) / 16) * (4 * ((H + 15) / 16 - 1) + (H - 16 * ((H + 15) / 16 - 1) + 3) / 4) +
           (nout <= 4 ? 0 : (4 * ((H + 15) / 16 - 1) + (H - 16 * ((H + 15) / 16 - 1) + 3) / 4));
}
__host__ __device__ constexpr double mfma_useful(int nin, int H, int NL, int nout) {
    return (double)(nin * H + (NL - 1) * H * H + (nout <= 4 ? 0 : H * nout)) / (64.0 * (double)mfma_per_tile(nin, H, NL, nout));
}
__host__ __device__ constexpr bool mfma_pays(int nin, int H, int NL, int nout) {
    return nout <= 16 && NL >= 1 && H >= 1 && mfma_useful(nin, H, NL, nout) >= NTC_MFMA_MIN_USEFUL;
}

template <class S, bool = S::kFixed && S::kUniform>
struct MfmaShape { static constexpr bool kOk = false; static constexpr double kUseful = 0.0; };
template <class S>
struct MfmaShape<S, true> {
    static constexpr int kIn = S::kNin, kH = S::kH, kNL = S::kNL, kNout = S::kNout;
    static constexpr int kHt = (kH + 15) / 16;            // 16-unit tiles of a hidden layer (the last one may be partial)
    static constexpr int kLastU = kH - 16 * (kHt - 1);    // units of the last tile (1 .. 16)
    static constexpr int kLastR = (kLastU + 3) / 4;       // its registers that hold units
    static constexpr int kKs1 = (kIn + 3) / 4;            // k-steps of the first layer (inputs padded with zeros)
    static constexpr int kKsH = 4 * (kHt - 1) + kLastR;   // k-steps of a layer fed by a hidden layer
    static constexpr int kDeep = kNL > 1 ? kNL - 1 : 1;
    static constexpr int kP = kH * kIn + kH + (kNL - 1) * (kH * kH + kH) + kNout * kH + kNout;   // parameters
    // matrix instructions per 16-pixel tile, and the fraction of their multiply-adds that are the model's
    static constexpr int kMfmaPerTile = kHt * kKs1 + (kNL - 1) * kHt * kKsH + (kNout <= 4 ? 0 : kKsH);
    static_assert(kMfmaPerTile == mfma_per_tile(kIn, kH, kNL, kNout), "the runtime count must follow the tile layout");
    static constexpr int kMacs = kIn * kH + (kNL - 1) * kH * kH + (kNout <= 4 ? 0 : kH * kNout);
    static constexpr double kUseful = (double)kMacs / (64.0 * kMfmaPerTile);
    static_assert(kUseful == mfma_useful(kIn, kH, kNL, kNout), "the runtime fraction must follow the tile layout");
    static constexpr bool kOk = mfma_pays(kIn, kH, kNL, kNout);
    // registers of hidden tile ot that hold units
    static constexpr int regs(int ot) { return ot == kHt - 1 ? kLastR : 4; }
    static constexpr bool partial(int ot) { return ot == kHt - 1 && kLastU < 16; }
};

// The unit in row i of hidden tile ot (a partial last tile: row 4g + r holds unit 4r + g of the tile).
template <class Q>
__host__ __device__ constexpr int unit_of(int ot, int i) { return Q::partial(ot) ? 16 * ot + 4 * (i & 3) + (i >> 2) : 16 * ot + i; }

// The hidden-layer input that lane group g feeds at k-step ks. Exact: the inputs in ascending order
// (k-step ks = inputs 4 ks .. 4 ks + 3; the activations are transposed to match). Otherwise the
// register of the previous layer's D layout as it stands: k-step 4 t + r takes register r of tile t,
// which lane group g holds as unit_of(t, 4 g + r).
template <class Q, bool Exact>
__host__ __device__ constexpr int hidden_input(int ks, int g) {
    if (Exact) return 4 * ks + g;
    const int t = (ks >> 2) < Q::kHt - 1 ? (ks >> 2) : Q::kHt - 1;
    return unit_of<Q>(t, 4 * g + (ks - 4 * t));
}

// Models with at most 4 outputs take their output layer on the VALU (valu_out_g): a matrix tile would
// spend 16 rows on them.
template <class S>
constexpr bool valu_out() { return MfmaShape<S>::kNout <= 4; }

// One member's parameters in operand layout.
template <class S>
struct MfmaWeights {
    using Q = MfmaShape<S>;
    float a1[Q::kHt][Q::kKs1];
    f4v c1[Q::kHt];
    float ah[Q::kDeep][Q::kHt][Q::kKsH];
    f4v ch[Q::kDeep][Q::kHt];
    float ao[Q::kKsH];                    // the output layer on the matrix cores
    f4v co;
    float wo[valu_out<S>() ? 4 : 1][Q::kKsH];   // the output layer on the VALU: output c's weight of the input this
    float bo[valu_out<S>() ? 4 : 1];            // lane group feeds at k-step ks; output c's bias in lane group 0
    // the pixel-per-lane output layer (mfma_out_own): the A operand of 4x4x1 step (ks, r) - in lane l, the
    // weight of output l % 4 for the input lane group r feeds at k-step ks - and the biases of outputs 0 .. 3
    float wo4[valu_out<S>() ? Q::kKsH : 1][4];
    f4v c4;
};

// Gathers a member's flat parameter vector (per layer W[out][in] row-major, then b[out]) into
// operand layout; lane = threadIdx.x % 64. Exact: the k-steps of a layer fed by a hidden layer take
// the inputs in ascending order (k-step ks = inputs 4 ks .. 4 ks + 3; the activations are transposed
// to match). Otherwise k-step 4 t + r takes the inputs in the order in which register r of hidden
// tile t holds them across the lane groups, and the activations feed the next layer untransposed:
// the same products, summed in another order. Padding units and inputs get zero weights: every lane
// reads a parameter (the index clamped to a valid one) and selects zero where it has none, so the gather
// takes no branches.
template <class S, bool Exact, class Get>
__device__ __forceinline__ void mfma_load_from(MfmaWeights<S>& W, const Get& w, int lane) {
    using Q = MfmaShape<S>;
    static_assert(!Exact || Q::kLastU == 16, "the ascending-order layout needs whole 16-unit tiles");
    constexpr int NIN = Q::kIn, H = Q::kH, NO = Q::kNout;
    const int i16 = lane & 15, g = lane >> 4;
    auto at = [&](bool ok, int k) { const float v = w(k); return ok ? v : 0.0f; };
#pragma unroll
    for (int ot = 0; ot < Q::kHt; ot++) {
        const int u = unit_of<Q>(ot, i16), uc = min(u, H - 1);
#pragma unroll
        for (int ks = 0; ks < Q::kKs1; ks++) {
            const int in = 4 * ks + g;
            W.a1[ot][ks] = at(in < NIN && u < H, uc * NIN + min(in, NIN - 1));
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int ur = unit_of<Q>(ot, 4 * g + r);
            W.c1[ot][r] = at(ur < H, H * NIN + min(ur, H - 1));
        }
    }
    int p = H * NIN + H;
#pragma unroll
    for (int l = 0; l < Q::kNL - 1; l++) {
#pragma unroll
        for (int ot = 0; ot < Q::kHt; ot++) {
            const int u = unit_of<Q>(ot, i16), uc = min(u, H - 1);
#pragma unroll
            for (int ks = 0; ks < Q::kKsH; ks++) {
                const int in = hidden_input<Q, Exact>(ks, g);
                W.ah[l][ot][ks] = at(u < H && in < H, p + uc * H + min(in, H - 1));
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int ur = unit_of<Q>(ot, 4 * g + r);
                W.ch[l][ot][r] = at(ur < H, p + H * H + min(ur, H - 1));
            }
        }
        p += H * H + H;
    }
    if constexpr (valu_out<S>()) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
#pragma unroll
            for (int ks = 0; ks < Q::kKsH; ks++) {
                const int in = hidden_input<Q, Exact>(ks, g);
                W.wo[c][ks] = c < NO ? at(in < H, p + c * H + min(in, H - 1)) : 0.0f;
            }
            W.bo[c] = c < NO ? at(g == 0, p + NO * H + c) : 0.0f;
            W.c4[c] = c < NO ? w(p + NO * H + c) : 0.0f;
        }
        const int oc = lane & 3, occ = min(oc, NO - 1);
#pragma unroll
        for (int ks = 0; ks < Q::kKsH; ks++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int in = hidden_input<Q, Exact>(ks, r);
                W.wo4[ks][r] = in < H ? at(oc < NO, p + occ * H + in) : 0.0f;
            }
    } else {
#pragma unroll
        for (int ks = 0; ks < Q::kKsH; ks++) {
            const int in = hidden_input<Q, Exact>(ks, g);
            W.ao[ks] = at(i16 < NO && in < H, p + min(i16, NO - 1) * H + min(in, H - 1));
        }
#pragma unroll
        for (int r = 0; r < 4; r++) W.co[r] = at(4 * g + r < NO, p + NO * H + min(4 * g + r, NO - 1));
    }
}

// parameter k of a member: a flat vector, or w0 + sg eps as one fused operation (main.cpp:1856)
struct ParamsAt {
    const float* w;
    __device__ __forceinline__ float operator()(int k) const { return w[k]; }
};
struct PerturbedParams {
    const float* w0; const float* eps; float sg;
    __device__ __forceinline__ float operator()(int k) const { return __builtin_fmaf(sg, eps[k], w0[k]); }
};

template <class S, bool Exact = true>
__device__ __forceinline__ void mfma_load(MfmaWeights<S>& W, const float* __restrict__ w, int lane) {
    mfma_load_from<S, Exact>(W, ParamsAt{ w }, lane);
}

// Output weights and biases times sc (the evaluations with the hardware sigmoid fold its -log2(e)
// into the output layer: the pre-activations come out as the exp2 argument).
template <class S>
__device__ __forceinline__ void scale_output(MfmaWeights<S>& W, float sc) {
    if constexpr (valu_out<S>()) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
#pragma unroll
            for (int ks = 0; ks < MfmaShape<S>::kKsH; ks++) W.wo[c][ks] *= sc;
            W.bo[c] *= sc;
            W.c4[c] *= sc;
        }
#pragma unroll
        for (int ks = 0; ks < MfmaShape<S>::kKsH; ks++)
#pragma unroll
            for (int r = 0; r < 4; r++) W.wo4[ks][r] *= sc;
    } else {
#pragma unroll
        for (int ks = 0; ks < MfmaShape<S>::kKsH; ks++) W.ao[ks] *= sc;
#pragma unroll
        for (int r = 0; r < 4; r++) W.co[r] *= sc;
    }
}

__device__ __forceinline__ f4v mfma4(float a, float b, f4v c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// v_mfma_f32_4x4x1_16b_f32: 16 independent 4 x 4 x 1 products, block b = lanes 4b .. 4b + 3:
// D[lane 4b + j][register i] = C[lane 4b + j][register i] + A[lane 4b + i] B[lane 4b + j] (measured on gfx950)
__device__ __forceinline__ f4v mfma4x4(float a, float b, f4v c) { return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0); }

// element (lane group g, register r) -> (lane group r, register g)
__device__ __forceinline__ void transpose4(const f4v& v, float* y) {
    const auto s02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[0]), __float_as_uint(v[2]), false, false);
    const auto s13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[1]), __float_as_uint(v[3]), false, false);
    const auto t01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
    const auto t23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
    y[0] = __uint_as_float(t01[0]); y[1] = __uint_as_float(t01[1]);
    y[2] = __uint_as_float(t23[0]); y[3] = __uint_as_float(t23[1]);
}

// Lane (t, j) holds the features f of pixel j of tile t (t = its lane group: a wave's 64 lanes build
// the features of 64 different pixels). The first layer's B operands of the four tiles: b[t][ks] in
// lane (g, j) = feature 4 ks + g of pixel j of tile t (zero past nin), one 4 x 4 transpose across
// the lane groups per k-step.
template <class S>
__device__ __forceinline__ void tiles_of(const float (&f)[S::kMaxIn], float (&b)[4][MfmaShape<S>::kKs1]) {
    using Q = MfmaShape<S>;
#pragma unroll
    for (int ks = 0; ks < Q::kKs1; ks++) {
        f4v v;
#pragma unroll
        for (int r = 0; r < 4; r++) v[r] = 4 * ks + r < Q::kIn ? f[4 * ks + r] : 0.0f;
        float y[4];
        transpose4(v, y);
#pragma unroll
        for (int t = 0; t < 4; t++) b[t][ks] = y[t];
    }
}

// How a kernel applies the activation of main.cpp:560, x > 0 ? x : leak x, to the matrix results. Every
// form propagates a NaN pre-activation as the reference's does (NaN > 0 is false and leak NaN is NaN),
// so a diverged member shows up as a NaN loss and a NaN update, never as a finite loss.
enum ActMode : int {
    kActAny = 0,    // any leak: a compare and a select
    kActMax = 1,    // 0 <= leak <= 1: max(x, leak x), bit for bit (also for signed zeros), one multiply and one maximum
                    // (a NaN x makes both operands NaN, so the maximum is NaN)
    kActFold = 3,   // 0 <= leak <= 1, with every hidden layer's weights and biases scaled by b = (1 + leak) / 2
                    // (scale_hidden): x' = b x and act = x' + c |x'| with c = (1 - leak) / (1 + leak), one fused
                    // multiply-add with an absolute-value operand - x for x > 0, leak x otherwise, within two
                    // roundings of the reference's value; for leak 0 (b = 1/2, c = 1) the value is the
                    // reference's exactly (scaling by 1/2 commutes with every rounding of the matrix chain;
                    // weights of magnitude below 2^-125 aside), except that a negative x gives +0 where the
                    // reference gives -0, which changes no sum it enters
};
// k: leak (kActAny, kActMax) or c (kActFold)
template <int Act>
__device__ __forceinline__ float act(float x, float k) {
    if constexpr (Act == kActMax) return fmaxf(x, k * x);
    else if constexpr (Act == kActFold) return __builtin_fmaf(k, __builtin_fabsf(x), x);
    else return x > 0.0f ? x : k * x;
}
// the activation constant k of act<Act> for a model's leak, and the hidden layers' weight scale b of kActFold
__host__ __device__ inline float act_k(int mode, float leak) { return mode == kActFold ? (1.0f - leak) / (1.0f + leak) : leak; }
__host__ __device__ inline float fold_scale(float leak) { return 0.5f * (1.0f + leak); }
// act_k for a model: kActFold's quotient comes divided from the host (DevModel::fold_c, the same IEEE division)
template <int Act>
__device__ __forceinline__ float act_k_of(const DevModel& m) { return Act == kActFold ? m.fold_c : m.leak; }

// Every hidden layer's weights and biases times b (kActFold).
template <class S>
__device__ __forceinline__ void scale_hidden(MfmaWeights<S>& W, float b) {
    using Q = MfmaShape<S>;
#pragma unroll
    for (int ot = 0; ot < Q::kHt; ot++) {
#pragma unroll
        for (int ks = 0; ks < Q::kKs1; ks++) W.a1[ot][ks] *= b;
#pragma unroll
        for (int r = 0; r < 4; r++) W.c1[ot][r] *= b;
    }
#pragma unroll
    for (int l = 0; l < Q::kNL - 1; l++)
#pragma unroll
        for (int ot = 0; ot < Q::kHt; ot++) {
#pragma unroll
            for (int ks = 0; ks < Q::kKsH; ks++) W.ah[l][ot][ks] *= b;
#pragma unroll
            for (int r = 0; r < 4; r++) W.ch[l][ot][r] *= b;
        }
}

// U independent 16-pixel tiles through the hidden layers (interleaved, so one tile's activations
// overlap the other's matrix operations): b1[u] = the first layer's B operands of tile u (input 4 ks +
// l / 16 of pixel l % 16, zero past nin); x[u] = the last hidden layer's activations of tile u as the
// next layer's B operands (k-step ks: hidden_input<Exact>(ks, l / 16) of pixel l % 16). Every lane of
// the wave must be active. Exact must match the weights' mfma_load; k is act_k(Act, leak).
template <class S, int U, int Act, bool Exact = true>
__device__ __forceinline__ void mfma_hidden(const MfmaWeights<S>& W, const float (&b1)[U][MfmaShape<S>::kKs1], float k,
                                            float (&x)[U][MfmaShape<S>::kKsH]) {
    using Q = MfmaShape<S>;
    {
        f4v acc[U][Q::kHt];
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int ot = 0; ot < Q::kHt; ot++) acc[u][ot] = W.c1[ot];
#pragma unroll
        for (int ks = 0; ks < Q::kKs1; ks++)
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int ot = 0; ot < Q::kHt; ot++) acc[u][ot] = mfma4(W.a1[ot][ks], b1[u][ks], acc[u][ot]);
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int ot = 0; ot < Q::kHt; ot++) {
#pragma unroll
                for (int r = 0; r < Q::regs(ot); r++) acc[u][ot][r] = act<Act>(acc[u][ot][r], k);
                if constexpr (Exact) transpose4(acc[u][ot], x[u] + 4 * ot);
                else {
#pragma unroll
                    for (int r = 0; r < Q::regs(ot); r++) x[u][4 * ot + r] = acc[u][ot][r];
                }
            }
    }
#pragma unroll
    for (int l = 0; l < Q::kNL - 1; l++) {
        f4v acc[U][Q::kHt];
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int ot = 0; ot < Q::kHt; ot++) acc[u][ot] = W.ch[l][ot];
#pragma unroll
        for (int ks = 0; ks < Q::kKsH; ks++)
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int ot = 0; ot < Q::kHt; ot++) acc[u][ot] = mfma4(W.ah[l][ot][ks], x[u][ks], acc[u][ot]);
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int ot = 0; ot < Q::kHt; ot++) {
#pragma unroll
                for (int r = 0; r < Q::regs(ot); r++) acc[u][ot][r] = act<Act>(acc[u][ot][r], k);
                if constexpr (Exact) transpose4(acc[u][ot], x[u] + 4 * ot);
                else {
#pragma unroll
                    for (int r = 0; r < Q::regs(ot); r++) x[u][4 * ot + r] = acc[u][ot][r];
                }
            }
    }
}
// ... and through the output layer on the matrix cores: the pre-activations of each tile in D layout
// (lane l, register r = output 4 (l / 16) + r of pixel l % 16).
template <class S, int U, int Act, bool Exact = true>
__device__ __forceinline__ void mfma_forward(const MfmaWeights<S>& W, const float (&b1)[U][MfmaShape<S>::kKs1], float k,
                                             f4v (&o)[U]) {
    using Q = MfmaShape<S>;
    float x[U][Q::kKsH];
    mfma_hidden<S, U, Act, Exact>(W, b1, k, x);
#pragma unroll
    for (int u = 0; u < U; u++) o[u] = W.co;
#pragma unroll
    for (int ks = 0; ks < Q::kKsH; ks++)
#pragma unroll
        for (int u = 0; u < U; u++) o[u] = mfma4(W.ao[ks], x[u][ks], o[u]);
}

// The output layer of four tiles for at most 4 outputs with the pixels in the lanes: x = the last hidden
// layer of tiles 0 .. 3 as mfma_hidden leaves it (lane (g, j), register ks of tile u = input
// hidden_input(ks, g) of pixel j). One 4 x 4 transpose across (lane group, tile) per k-step gives lane
// (g, j) every input of pixel j of tile g (register r: input hidden_input(ks, r)); then each input is one
// 4x4x1 step whose A operand holds output l % 4's weight of it, so the block of lanes 4b .. 4b + 3 adds
// w[i][in] x[in] of its four pixels into output i: lane (g, j) ends with the pre-activations of outputs
// 0 .. 3 of its own pixel (bias first, then the inputs in k-step order; outputs past nout are zero).
// 16 4x4x1 steps (8 cycles each) and 16 lane swaps per 16-unit tile set, where the VALU layer spends
// 4 x (3 x 4 fused multiply-adds + its reduce-scatter) and one sigmoid per lane and tile.
template <class S>
__device__ __forceinline__ f4v mfma_out_own(const MfmaWeights<S>& W, const float (&x)[4][MfmaShape<S>::kKsH]) {
    static_assert(valu_out<S>(), "at most 4 outputs");
    // two independent chains (inputs of registers 0, 1 and 2, 3), added at the end
    f4v o = W.c4, o2 = { 0.0f, 0.0f, 0.0f, 0.0f };
#pragma unroll
    for (int ks = 0; ks < MfmaShape<S>::kKsH; ks++) {
        f4v v;
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = x[u][ks];
        float y[4];
        transpose4(v, y);
        o = mfma4x4(W.wo4[ks][0], y[0], o);
        o2 = mfma4x4(W.wo4[ks][2], y[2], o2);
        o = mfma4x4(W.wo4[ks][1], y[1], o);
        o2 = mfma4x4(W.wo4[ks][3], y[3], o2);
    }
#pragma unroll
    for (int r = 0; r < MfmaShape<S>::kNout; r++) o[r] += o2[r];
    return o;
}

// mfma_out_own with the (lane group, tile) transpose through LDS rows of the wave's own instead of lane
// swaps (each swap costs the SIMD about three VALU issue slots; the LDS moves issue beside other waves'
// matrix and VALU work): lane (g, j) writes register ks of tile u to row (u, j), column 4 g + ks, and
// reads row (g, j) back, column 4 r + ks being what the swaps leave in its register r at k-step ks. Rows
// are kOwnRow floats apart (20: the 16 lanes of a group write and read 16-byte pieces in 16 distinct
// groups of four banks). A wave's LDS operations complete in program order, so its reads see its writes
// and the next pass's writes come after these reads: no barrier (the fences only keep the compiler
// from reordering them). The same products, summed in the same order as mfma_out_own.
constexpr int kOwnRow = 20, kOwnWave = 4 * 16 * kOwnRow;
template <class S>
__device__ __forceinline__ f4v mfma_out_own_lds(const MfmaWeights<S>& W, const float (&x)[4][MfmaShape<S>::kKsH],
                                                float* __restrict__ t, int g, int j) {
    static_assert(valu_out<S>() && MfmaShape<S>::kKsH <= 4, "at most 4 outputs, one 16-unit tile");
    constexpr int KS = MfmaShape<S>::kKsH;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        f4v v = { 0.0f, 0.0f, 0.0f, 0.0f };
#pragma unroll
        for (int ks = 0; ks < KS; ks++) v[ks] = x[u][ks];
        *reinterpret_cast<f4v*>(t + (u * 16 + j) * kOwnRow + 4 * g) = v;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    f4v y[4];
#pragma unroll
    for (int r = 0; r < 4; r++) y[r] = *reinterpret_cast<const f4v*>(t + (g * 16 + j) * kOwnRow + 4 * r);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    f4v o = W.c4, o2 = { 0.0f, 0.0f, 0.0f, 0.0f };
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        o = mfma4x4(W.wo4[ks][0], y[0][ks], o);
        o2 = mfma4x4(W.wo4[ks][2], y[2][ks], o2);
        o = mfma4x4(W.wo4[ks][1], y[1][ks], o);
        o2 = mfma4x4(W.wo4[ks][3], y[3][ks], o2);
    }
#pragma unroll
    for (int r = 0; r < MfmaShape<S>::kNout; r++) o[r] += o2[r];
    return o;
}

// The output layer on the VALU for at most 4 outputs: lane (g, j) forms the partial sums of every
// output over the hidden inputs it holds (x, the last hidden layer in the order mfma_hidden leaves it),
// and a reduce-scatter over the four lane groups - two permlane32 swaps, one permlane16 swap, three adds
// - leaves output g of pixel j in lane (g, j), summed (g0 + g2) + (g1 + g3) over the lane groups' parts.
// Lane groups g >= nout hold zeros.
template <class S>
__device__ __forceinline__ float valu_out_g(const MfmaWeights<S>& W, const float (&x)[MfmaShape<S>::kKsH]) {
    static_assert(valu_out<S>(), "at most 4 outputs");
    constexpr int NO = MfmaShape<S>::kNout;
    float p[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        p[c] = W.bo[c];
        if (c < NO) {
#pragma unroll
            for (int ks = 0; ks < MfmaShape<S>::kKsH; ks++) p[c] = __builtin_fmaf(W.wo[c][ks], x[ks], p[c]);
        }
    }
    const auto s02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(p[0]), __float_as_uint(p[2]), false, false);
    const auto s13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(p[1]), __float_as_uint(p[3]), false, false);
    const float q02 = __uint_as_float(s02[0]) + __uint_as_float(s02[1]);   // groups 0, 1: output 0; groups 2, 3: output 2
    const float q13 = __uint_as_float(s13[0]) + __uint_as_float(s13[1]);   // groups 0, 1: output 1; groups 2, 3: output 3
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(q02), __float_as_uint(q13), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// valu_out_g with the reduce-scatter through kVoTile floats of the wave's own LDS (t) instead of lane swaps
// (cheaper in VALU issue slots, as for mfma_out_own_lds): lane (g, j) writes its partial of output c to row
// j, column 4 c + g (rows kOwnRow floats apart: conflict-free), then reads row j's columns 4 g .. 4 g + 3 -
// output g's four partials - and adds them as valu_out_g does, (g0 + g2) + (g1 + g3): the same value bit for bit.
constexpr int kVoTile = 16 * kOwnRow;
template <class S>
__device__ __forceinline__ float valu_out_g_lds(const MfmaWeights<S>& W, const float (&x)[MfmaShape<S>::kKsH], float* __restrict__ t,
                                                int g, int j) {
    static_assert(valu_out<S>(), "at most 4 outputs");
    constexpr int NO = MfmaShape<S>::kNout;
    float p[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        p[c] = W.bo[c];
        if (c < NO) {
#pragma unroll
            for (int ks = 0; ks < MfmaShape<S>::kKsH; ks++) p[c] = __builtin_fmaf(W.wo[c][ks], x[ks], p[c]);
        }
    }
#pragma unroll
    for (int c = 0; c < 4; c++) t[j * kOwnRow + 4 * c + g] = p[c];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const f4v v = *reinterpret_cast<const f4v*>(t + j * kOwnRow + 4 * g);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    return (v[0] + v[2]) + (v[1] + v[3]);
}

// Wave-local LDS exchanges in place of lane swaps (a wave's LDS operations complete in program order, so
// no barrier; the fences only keep the compiler from moving them across each other).
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// tiles_of through kTilesLds<S> floats of the wave's LDS: lane (t, j) writes feature 4 ks + r of its pixel
// to [r][ks][j][t], lane (g, j) reads [g][ks][j][0 .. 3] = b[0 .. 3][ks] (every access conflict-free).
template <class S>
constexpr int kTilesLds = 4 * MfmaShape<S>::kKs1 * 64;
template <class S>
__device__ __forceinline__ void tiles_of_lds(const float (&f)[S::kMaxIn], float (&b)[4][MfmaShape<S>::kKs1], float* __restrict__ t,
                                             int g, int j) {
    using Q = MfmaShape<S>;
#pragma unroll
    for (int ks = 0; ks < Q::kKs1; ks++)
#pragma unroll
        for (int r = 0; r < 4; r++) t[((r * Q::kKs1 + ks) * 16 + j) * 4 + g] = 4 * ks + r < Q::kIn ? f[4 * ks + r] : 0.0f;
    wave_lds_fence();
#pragma unroll
    for (int ks = 0; ks < Q::kKs1; ks++) {
        const f4v v = *reinterpret_cast<const f4v*>(t + ((g * Q::kKs1 + ks) * 16 + j) * 4);
#pragma unroll
        for (int tt = 0; tt < 4; tt++) b[tt][ks] = v[tt];
    }
    wave_lds_fence();
}

// The sums of a and of b over the four lane groups of each pixel, in every one of them, added as group_sum_f
// adds them, (g0 + g2) + (g1 + g3), through kSumsLds floats of the wave's LDS (rows kOwnRow apart).
constexpr int kSumsLds = 16 * kOwnRow;
__device__ __forceinline__ void group_sums_lds(float a, float b, float* __restrict__ t, int g, int j, float& sa, float& sb) {
    t[j * kOwnRow + g] = a;
    t[j * kOwnRow + 4 + g] = b;
    wave_lds_fence();
    const f4v va = *reinterpret_cast<const f4v*>(t + j * kOwnRow), vb = *reinterpret_cast<const f4v*>(t + j * kOwnRow + 4);
    wave_lds_fence();
    sa = (va[0] + va[2]) + (va[1] + va[3]);
    sb = (vb[0] + vb[2]) + (vb[1] + vb[3]);
}


// ---- per-pixel error across the output tile
// Lane (g, j) holds the output units 4 g + r of pixel j; the reference sums a pixel's channels
// in ascending order. The running sum starts in lane group 0, each group adds its (up to) four
// channels and hands the sum to the next group (ds_bpermute from lane - 16); the result is valid
// in the lanes of group (NO - 1) / 4.
__device__ __forceinline__ int lane_below_addr(int lane) { return ((lane - 16) & 63) << 2; }

// decode_err (main.cpp:1731-1732): e = fma(cw, d d, e), float
template <int NO>
__device__ __forceinline__ float chain_err_f(const float (&dd)[4], const float (&cw)[4], int lane) {
    constexpr int NG = (NO + 3) / 4;
    const int from = lane_below_addr(lane);
    float e = 0.0f;
#pragma unroll
    for (int gg = 0; gg < NG; gg++) {
        if (gg > 0) e = __int_as_float(__builtin_amdgcn_ds_bpermute(from, __float_as_int(e)));
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (4 * gg + r < NO) e = __builtin_fmaf(cw[r], dd[r], e);
    }
    return e;
}

// The sum of v over the four lane groups of each pixel (lanes j, j + 16, j + 32, j + 48), in every
// one of them: (g0 + g2) + (g1 + g3), from two permlane swaps of each half of the double (no LDS).
__device__ __forceinline__ double group_sum_d(double v) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)b, hi = (unsigned)(b >> 32);
    auto join = [](unsigned l, unsigned h) { return __longlong_as_double((long long)(((unsigned long long)h << 32) | l)); };
    const auto l32 = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto h32 = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    const double s = join(l32[0], h32[0]) + join(l32[1], h32[1]);   // rows: g0 + g2, g1 + g3, g0 + g2, g1 + g3
    const unsigned long long sb = (unsigned long long)__double_as_longlong(s);
    const auto l16 = __builtin_amdgcn_permlane16_swap((unsigned)sb, (unsigned)sb, false, false);
    const auto h16 = __builtin_amdgcn_permlane16_swap((unsigned)(sb >> 32), (unsigned)(sb >> 32), false, false);
    return join(l16[0], h16[0]) + join(l16[1], h16[1]);
}

// The float sum of v over the four lane groups of each pixel, in every one of them: (g0 + g2) + (g1 + g3).
__device__ __forceinline__ float group_sum_f(float v) {
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float s = __uint_as_float(h[0]) + __uint_as_float(h[1]);   // rows: g0 + g2, g1 + g3, g0 + g2, g1 + g3
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// loss_subset's per-pixel terms (main.cpp:1747): s += (double)(cw (d d)), double
template <int NO>
__device__ __forceinline__ double chain_err_d(const float (&dd)[4], const float (&cw)[4], int lane) {
    constexpr int NG = (NO + 3) / 4;
    const int from = lane_below_addr(lane);
    double e = 0.0;
#pragma unroll
    for (int gg = 0; gg < NG; gg++) {
        if (gg > 0) {
            const long long b = __double_as_longlong(e);
            const int lo = __builtin_amdgcn_ds_bpermute(from, (int)(b & 0xFFFFFFFFll));
            const int hi = __builtin_amdgcn_ds_bpermute(from, (int)(b >> 32));
            e = __longlong_as_double(((long long)hi << 32) | (long long)(unsigned)lo);
        }
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (4 * gg + r < NO) e += (double)__fmul_rn(cw[r], dd[r]);
    }
    return e;
}

// the channel weights of this lane's output units (0 past nout)
template <int NO>
__device__ __forceinline__ void lane_cw(const float* cwm, int g, float (&cw)[4]) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
        cw[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < NO; c++) if (4 * g + r == c) cw[r] = cwm[c];
    }
}

}   // namespace ntc_hip
