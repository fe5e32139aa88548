// The MLP of the fixed shapes on the FP32 matrix cores of gfx950 (v_mfma_f32_16x16x4f32), as the training
// kernels of kern_pop.hpp evaluate it.
//
// One wave evaluates one member's MLP on a tile of 16 pixels at a time, with the member's
// parameters held in VGPRs in the instruction's operand layout:
//   A (16 x 4)  lane l holds A[l % 16][l / 16]        weights W[out][in]: out = 16 ot + l % 16
//   B (4 x 16)  lane l holds B[l / 16][l % 16]        activations of pixel l % 16
//   C/D (16x16) lane l, register r holds D[4 (l / 16) + r][l % 16]
// On gfx950 this instruction computes D = C then D = fma(A[.][k], B[k][.], D) for k = 0..3 in
// order, each step rounded (measured against host fmaf chains on 1 M random values, including
// subnormal operands, with no difference): with C = the bias, every unit is a chain of fused
// multiply-adds over its inputs, as the reference's s = b[j]; s = fma(w[j][i], a[i], s) is
// (main.cpp:603-627), with the inputs of a layer fed by a hidden layer taken in another order.
//
// A layer's output comes back in the D layout (lane group g holds units 4g + r of a 16-unit tile),
// and that is how the next layer takes it: k-step 4 t + r takes register r of hidden tile t, which
// lane group g holds as unit 4 g + r (hidden_input), so the weights are gathered in that order and the
// activations feed the next layer untransposed - the same products, summed in another order than the
// reference's ascending one (within a few roundings of it).
//
// Hidden widths that are not a multiple of 16 pad the last tile with zero weights and biases. Its
// rows are ordered so that the units sit in the first registers of the four lane groups (row 4g + r
// holds unit 4r + g of the tile): the registers past the last unit hold padding only, and the next
// layer skips their k-steps (36 units: 9 k-steps, not 12). Padded rows compute fma(0, x, 0) chains
// and activate to zero, so the real units are unchanged.
//
// Data that has to move between lane groups (transposes, reduce-scatters, a pixel's sums over its four
// lanes) goes through LDS rows of the wave's own rather than through lane swaps: a v_permlane32_swap or
// v_permlane16_swap costs the SIMD about three VALU issue slots, while LDS reads and writes issue on the
// LDS pipe beside other waves' matrix and VALU work. A wave's LDS operations complete in program order,
// so its reads see its writes and no barrier is needed.
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

// The hidden-layer input that lane group g feeds at k-step ks: the register of the previous layer's D
// layout as it stands - k-step 4 t + r takes register r of tile t, which lane group g holds as
// unit_of(t, 4 g + r).
template <class Q>
__host__ __device__ constexpr int hidden_input(int ks, int g) {
    const int t = (ks >> 2) < Q::kHt - 1 ? (ks >> 2) : Q::kHt - 1;
    return unit_of<Q>(t, 4 * g + (ks - 4 * t));
}

// Models with at most 4 outputs take their output layer on the VALU (valu_out_g): a matrix tile would
// spend 16 rows on them.
template <class S>
constexpr bool valu_out() { return MfmaShape<S>::kNout <= 4; }

// The output layer on the matrix cores (more than 4 outputs): row 4 g + r of the output tile holds output
// kOutR g + r for r < kOutR = ceil(nout / 4), the other rows padding, so each lane's outputs sit in its first
// kOutR registers and the rest of every lane's registers hold padding only (12 outputs: three registers of
// every lane group, not four registers of three groups): the sigmoid and error terms skip whole registers.
// out_at = the output in register r of lane group g, or -1 for padding.
template <class S>
constexpr int out_regs() { return (MfmaShape<S>::kNout + 3) / 4; }
template <class S>
__host__ __device__ constexpr int out_at(int g, int r) {
    return r < out_regs<S>() && out_regs<S>() * g + r < MfmaShape<S>::kNout ? out_regs<S>() * g + r : -1;
}

// One member's parameters in operand layout.
template <class S>
struct MfmaWeights {
    using Q = MfmaShape<S>;
    float a1[Q::kHt][Q::kKs1];
    f4v c1[Q::kHt];
    float ah[Q::kDeep][Q::kHt][Q::kKsH];
    f4v ch[Q::kDeep][Q::kHt];
    float ao[Q::kKsH];                    // the output layer on the matrix cores (rows as out_at)
    f4v co;
    float wo[valu_out<S>() ? 4 : 1][Q::kKsH];   // the output layer on the VALU: output c's weight of the input this
    float bo[valu_out<S>() ? 4 : 1];            // lane group feeds at k-step ks; output c's bias in lane group 0
    // the pixel-per-lane output layer (mfma_out_own): the A operand of 4x4x1 step (ks, r) - in lane l, the
    // weight of output l % 4 for the input lane group r feeds at k-step ks - and the biases of outputs 0 .. 3
    float wo4[valu_out<S>() ? Q::kKsH : 1][4];
    f4v c4;
};

// The order in which the first layer's k-steps take the model's inputs: position p of the operand rows holds
// input InMap::map(p) (the identity: the reference's input order).
struct InIdentity {
    __host__ __device__ static constexpr int map(int p) { return p; }
};

// Gathers a member's flat parameter vector (per layer W[out][in] row-major, then b[out]) into
// operand layout; lane = threadIdx.x % 64. Padding units, inputs and outputs get zero weights: every lane
// reads a parameter (the index clamped to a valid one) and selects zero where it has none, so the gather
// takes no branches.
template <class S, class Get, class InMap = InIdentity>
__device__ __forceinline__ void mfma_load_from(MfmaWeights<S>& W, const Get& w, int lane) {
    using Q = MfmaShape<S>;
    constexpr int NIN = Q::kIn, H = Q::kH, NO = Q::kNout;
    const int i16 = lane & 15, g = lane >> 4;
    auto at = [&](bool ok, int k) { const float v = w(k); return ok ? v : 0.0f; };
#pragma unroll
    for (int ot = 0; ot < Q::kHt; ot++) {
        const int u = unit_of<Q>(ot, i16), uc = min(u, H - 1);
#pragma unroll
        for (int ks = 0; ks < Q::kKs1; ks++) {
            const int pos = 4 * ks + g, in = pos < NIN ? InMap::map(pos) : pos;
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
                const int in = hidden_input<Q>(ks, g);
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
                const int in = hidden_input<Q>(ks, g);
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
                const int in = hidden_input<Q>(ks, r);
                W.wo4[ks][r] = in < H ? at(oc < NO, p + occ * H + in) : 0.0f;
            }
    } else {
        const int orow = out_at<S>(i16 >> 2, i16 & 3);   // the output in row i16 of the output tile
#pragma unroll
        for (int ks = 0; ks < Q::kKsH; ks++) {
            const int in = hidden_input<Q>(ks, g);
            W.ao[ks] = at(orow >= 0 && in < H, p + max(orow, 0) * H + min(in, H - 1));
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int oc = out_at<S>(g, r);
            W.co[r] = at(oc >= 0, p + NO * H + max(oc, 0));
        }
    }
}

// parameter k of a member's flat vector
struct ParamsAt {
    const float* w;
    __device__ __forceinline__ float operator()(int k) const { return w[k]; }
};

template <class S, class InMap = InIdentity>
__device__ __forceinline__ void mfma_load(MfmaWeights<S>& W, const float* __restrict__ w, int lane) {
    mfma_load_from<S, ParamsAt, InMap>(W, ParamsAt{ w }, lane);
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
// next layer's B operands (k-step ks: hidden_input(ks, l / 16) of pixel l % 16). Every lane of the wave
// must be active. k is act_k(Act, leak).
// mfma_hidden in two parts. The first layer's pre-activations of U tiles in D layout (acc[u][ot]: hidden tile ot).
template <class S, int U>
__device__ __forceinline__ void mfma_layer1(const MfmaWeights<S>& W, const float (&b1)[U][MfmaShape<S>::kKs1],
                                            f4v (&acc)[U][MfmaShape<S>::kHt]) {
    using Q = MfmaShape<S>;
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
}
// ... and from those pre-activations through the activation and the other hidden layers (x as mfma_hidden
// leaves it).
template <class S, int U, int Act>
__device__ __forceinline__ void mfma_hidden_from1(const MfmaWeights<S>& W, const f4v (&acc1)[U][MfmaShape<S>::kHt], float k,
                                                  float (&x)[U][MfmaShape<S>::kKsH]) {
    using Q = MfmaShape<S>;
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
        for (int ot = 0; ot < Q::kHt; ot++)
#pragma unroll
            for (int r = 0; r < Q::regs(ot); r++) x[u][4 * ot + r] = act<Act>(acc1[u][ot][r], k);
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
            for (int ot = 0; ot < Q::kHt; ot++)
#pragma unroll
                for (int r = 0; r < Q::regs(ot); r++) x[u][4 * ot + r] = act<Act>(acc[u][ot][r], k);
    }
}
template <class S, int U, int Act>
__device__ __forceinline__ void mfma_hidden(const MfmaWeights<S>& W, const float (&b1)[U][MfmaShape<S>::kKs1], float k,
                                            float (&x)[U][MfmaShape<S>::kKsH]) {
    f4v acc[U][MfmaShape<S>::kHt];
    mfma_layer1<S, U>(W, b1, acc);
    mfma_hidden_from1<S, U, Act>(W, acc, k, x);
}
// The output layer on the matrix cores: the pre-activations of each tile in D layout (lane l, register r =
// output out_at(l / 16, r) of pixel l % 16).
template <class S, int U>
__device__ __forceinline__ void mfma_output(const MfmaWeights<S>& W, const float (&x)[U][MfmaShape<S>::kKsH], f4v (&o)[U]) {
#pragma unroll
    for (int u = 0; u < U; u++) o[u] = W.co;
#pragma unroll
    for (int ks = 0; ks < MfmaShape<S>::kKsH; ks++)
#pragma unroll
        for (int u = 0; u < U; u++) o[u] = mfma4(W.ao[ks], x[u][ks], o[u]);
}
// The whole MLP of U tiles from the first layer's B operands to the output pre-activations.
template <class S, int U, int Act>
__device__ __forceinline__ void mfma_forward(const MfmaWeights<S>& W, const float (&b1)[U][MfmaShape<S>::kKs1], float k,
                                             f4v (&o)[U]) {
    float x[U][MfmaShape<S>::kKsH];
    mfma_hidden<S, U, Act>(W, b1, k, x);
    mfma_output<S, U>(W, x, o);
}

// ---- exchanges between lane groups through the wave's own LDS rows
// Rows are kOwnRow floats apart: the 16 lanes of a group, each reading or writing 4 or 16 bytes of its own
// row, hit distinct banks.
constexpr int kOwnRow = 20;

// a wave's LDS operations complete in program order; the fences only keep the compiler from moving the
// reads above the writes (or the next writes above the reads)
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The output layer of four tiles for at most 4 outputs and one 16-unit hidden tile with the pixels in the
// lanes: x = the last hidden layer of tiles 0 .. 3 as mfma_hidden leaves it (lane (g, j), register ks of
// tile u = input hidden_input(ks, g) of pixel j). Lane (g, j) writes register ks of tile u to row (u, j),
// column 4 g + ks of t (kOwnWave floats), and reads row (g, j): every input of pixel j of tile g, column
// 4 r + ks = input hidden_input(ks, r). Each input is then one 4x4x1 step whose A operand holds output
// l % 4's weight of it, so the block of lanes 4b .. 4b + 3 adds w[i][in] x[in] of its four pixels into
// output i: lane (g, j) ends with the pre-activations of outputs 0 .. 3 of its own pixel (bias first, then
// the inputs in k-step order, in two chains added at the end; outputs past nout are zero). 16 4x4x1 steps
// (8 cycles each) per four tiles, where the VALU layer spends 4 x (3 x 4 fused multiply-adds + its
// reduce-scatter) and one sigmoid per lane and tile.
constexpr int kOwnWave = 4 * 16 * kOwnRow;
template <class S>
__device__ __forceinline__ f4v mfma_out_own(const MfmaWeights<S>& W, const float (&x)[4][MfmaShape<S>::kKsH],
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
    wave_lds_fence();
    f4v y[4];
#pragma unroll
    for (int r = 0; r < 4; r++) y[r] = *reinterpret_cast<const f4v*>(t + (g * 16 + j) * kOwnRow + 4 * r);
    wave_lds_fence();
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
// writes them to row j, columns 4 c + g of t (kVoTile floats), and reads back row j's columns 4 g .. 4 g + 3:
// the four lane groups' parts of output g, which it adds as (g0 + g2) + (g1 + g3). Output g of pixel j ends in
// lane (g, j); lane groups g >= nout hold zeros.
constexpr int kVoTile = 16 * kOwnRow;
template <class S>
__device__ __forceinline__ float valu_out_g(const MfmaWeights<S>& W, const float (&x)[MfmaShape<S>::kKsH], float* __restrict__ t,
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
    wave_lds_fence();
    const f4v v = *reinterpret_cast<const f4v*>(t + j * kOwnRow + 4 * g);
    wave_lds_fence();
    return (v[0] + v[2]) + (v[1] + v[3]);
}

// Lane (t, j) holds the features f of pixel j of tile t (t = its lane group: a wave's 64 lanes build the
// features of 64 different pixels). The first layer's B operands of the four tiles: b[t][ks] in lane (g, j)
// = feature 4 ks + g of pixel j of tile t (zero past nin). Through kTilesLds<S> floats of the wave's LDS:
// lane (t, j) writes feature 4 ks + r of its pixel to [r][ks][j][t], lane (g, j) reads [g][ks][j][0 .. 3].
template <class S>
constexpr int kTilesLds = 4 * MfmaShape<S>::kKs1 * 64;
template <class S>
__device__ __forceinline__ void tiles_of(const float (&f)[S::kMaxIn], float (&b)[4][MfmaShape<S>::kKs1], float* __restrict__ t,
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

// tiles_of for NK k-steps of values f[0 .. N) (zero from N on): b[t][ks] in lane (g, j) = value 4 ks + g of the
// pixel that lane (t, j) built, through 4 NK 64 floats of the wave's LDS.
template <int NK, int N>
__device__ __forceinline__ void tiles_of_n(const float (&f)[N], float (&b)[4][NK], float* __restrict__ t, int g, int j) {
#pragma unroll
    for (int ks = 0; ks < NK; ks++)
#pragma unroll
        for (int r = 0; r < 4; r++) t[((r * NK + ks) * 16 + j) * 4 + g] = 4 * ks + r < N ? f[4 * ks + r] : 0.0f;
    wave_lds_fence();
#pragma unroll
    for (int ks = 0; ks < NK; ks++) {
        const f4v v = *reinterpret_cast<const f4v*>(t + ((g * NK + ks) * 16 + j) * 4);
#pragma unroll
        for (int tt = 0; tt < 4; tt++) b[tt][ks] = v[tt];
    }
    wave_lds_fence();
}

// The sums of a and of b over the four lane groups of each pixel (lanes j, j + 16, j + 32, j + 48), in every
// one of them, added as (g0 + g2) + (g1 + g3), through kSumsLds floats of the wave's LDS.
constexpr int kSumsLds = 16 * kOwnRow;
__device__ __forceinline__ void group_sums(float a, float b, float* __restrict__ t, int g, int j, float& sa, float& sb) {
    t[j * kOwnRow + g] = a;
    t[j * kOwnRow + 4 + g] = b;
    wave_lds_fence();
    const f4v va = *reinterpret_cast<const f4v*>(t + j * kOwnRow), vb = *reinterpret_cast<const f4v*>(t + j * kOwnRow + 4);
    wave_lds_fence();
    sa = (va[0] + va[2]) + (va[1] + va[3]);
    sb = (vb[0] + vb[2]) + (vb[1] + vb[3]);
}

// the channel weights of this lane's output registers on the matrix output layer (out_at; 0 for padding)
template <class S>
__device__ __forceinline__ void lane_cw(const float* cwm, int g, float (&cw)[4]) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
        cw[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < MfmaShape<S>::kNout; c++) if (out_at<S>(g, r) == c) cw[r] = cwm[c];
    }
}

}   // namespace ntc_hip
