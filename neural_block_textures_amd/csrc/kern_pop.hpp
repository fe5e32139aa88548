// Device code only (compiled into libntc_hip.so for the fixed shapes of shapes.hpp, and by hipRTC at
// init for the shape of a model that is none of them, jit.cpp); the launchers are in kernels_pop.hip.
//
// The population evaluation (MlpTrainer::step's member losses, main.cpp:1848-1861) on the FP32
// matrix cores of gfx950, for the fixed shapes the matrix cores pay off for (MfmaShape::kOk) and
// 0 <= leak <= 1; other models use the VALU kernel of kernels_mlp.hip. In an ES step the kernel
// stages the pair's perturbed weights itself (no member weight sets in memory).
//
// On this chip an FP32 matrix instruction and a VALU instruction do not run concurrently on a
// SIMD (a 16x16x4 f32 step costs 32 cycles, a VALU instruction 4, and their mixes take the sum),
// so everything around the matrix operations is counted in instructions: the activation is one
// instruction (kActFold's fused multiply-add on hidden layers whose weights were scaled by
// (1 + leak) / 2 when the member's weights were staged, which propagates a NaN as the reference's
// activation does); a hidden layer's outputs feed the next layer in the order
// the matrix instruction leaves them (no transpose; each unit's sum takes its inputs in another
// order than the reference's ascending one); the sigmoid is the hardware exp2 and reciprocal, its
// -log2(e) folded into the output layer; a lane's channel terms cw d d are fused multiply-adds in float
// over the tiles a wave evaluates at once, then added into a double; tile
// inputs are buffer loads with a loop-invariant lane offset and the tile's offset in an SGPR. Member
// losses stay within 1e-5 relative of the reference's (they are not bit-identical here anyway:
// the sigmoid differs in the last bits).
//
// Block (pair, chunk) has four waves: wave w evaluates member 2 pair + (w & 1) on the 16-slot
// tiles 2 j + (w >> 1) of the chunk, two tiles at a time, the next two tiles' inputs loading
// while the current ones compute. Each lane adds the float terms cw (d d) (main.cpp:1747) of its
// output channels into a double; the two waves of a member are added in a fixed order.
#pragma once
#include "mfma_mlp.hpp"

namespace ntc_hip {

constexpr int kPopWaves = 4;
// Models with at most 4 outputs and one 16-unit hidden tile take the pixel-per-lane output layer
// (mfma_out_own): four tiles per pass, exchanged through the wave's LDS so that every lane holds all hidden
// units of one pixel, then v_mfma_f32_4x4x1_16b_f32 steps leave that pixel's outputs in its own registers.
template <class S>
constexpr bool pop_own() { return valu_out<S>() && MfmaShape<S>::kHt == 1; }
// 16-slot tiles a wave evaluates at once (independent chains of matrix instructions; two for the other
// shapes: the 64-wide models then hold 236 VGPRs at two waves per SIMD)
template <class S>
constexpr int pop_u() { return pop_own<S>() ? 4 : 2; }

// The minibatch arrays are read through raw buffers (buffer_of): loads take a loop-invariant 32-bit lane
// offset (VGPR) and the tile's byte offset (SGPR), so no address arithmetic per load. num_records = the
// allocation (every read stays inside it: minibatch_rows(nin) feature rows, those past nin zero, and
// kMinibatchSlack floats past the last row of each array).

// The targets a lane needs per tile: the pixel-per-lane output layer leaves every output of the lane's
// own pixel in the lane (its nout targets, once per pass); models with at most 4 outputs otherwise take
// their output layer on the VALU (valu_out_g), which leaves output g of pixel j in lane (g, j): one
// target per tile; otherwise the D layout's out_regs per tile (outputs out_at(g, r)).
template <class S>
constexpr int pop_nt() { return pop_own<S>() ? MfmaShape<S>::kNout : (valu_out<S>() ? 1 : out_regs<S>()); }
template <class S>
constexpr int pop_tt() { return pop_own<S>() ? 1 : pop_u<S>(); }

// Whether the loop runs two whole passes as one straight-line block (so that one pass's output stage can
// overlap the next pass's hidden layers), masking only the passes at the chunk's end: measured on the
// MI355X, 3.5% faster for the 3-output 32-wide shapes (dct512: 0.425 -> 0.410 ms), 0.5-2% slower for the
// 12-output and the pixel-per-lane shapes (one more occupancy step of registers, or nothing to overlap).
template <class S>
constexpr bool pop_pairs_whole() { return valu_out<S>() && !pop_own<S>(); }

// a compile-time flag handed to a generic lambda
template <bool B>
struct WholeTag { static constexpr bool value = B; };

template <class S>
struct PopTileIn {
    float b1[pop_u<S>()][MfmaShape<S>::kKs1];
    float t[pop_tt<S>()][pop_nt<S>()];
};

// Inputs of tiles j .. j + U - 1 of this wave: soff = byte offset of tile j's first slot (uniform);
// tile u sits 32 slots further per u. With the pixel-per-lane output layer, lane (g, i) loads the
// targets of pixel i of tile g (its lane offsets include the 32 g slots).
template <class S>
__device__ __forceinline__ void pop_load(PopTileIn<S>& in, __amdgpu_buffer_rsrc_t rf, __amdgpu_buffer_rsrc_t rt, uint32_t soff,
                                         const uint32_t (&fo)[MfmaShape<S>::kKs1], const uint32_t (&to)[pop_nt<S>()]) {
    using Q = MfmaShape<S>;
#pragma unroll
    for (int u = 0; u < pop_u<S>(); u++) {
        const uint32_t so = (uint32_t)__builtin_amdgcn_readfirstlane((int)(soff + 128u * u));   // uniform: an SGPR
#pragma unroll
        for (int ks = 0; ks < Q::kKs1; ks++) in.b1[u][ks] = buffer_f32(rf, fo[ks], so);
        if constexpr (!pop_own<S>()) {
#pragma unroll
            for (int r = 0; r < pop_nt<S>(); r++) in.t[u][r] = buffer_f32(rt, to[r], so);
        }
    }
    if constexpr (pop_own<S>()) {
        const uint32_t so = (uint32_t)__builtin_amdgcn_readfirstlane((int)soff);
#pragma unroll
        for (int c = 0; c < pop_nt<S>(); c++) in.t[0][c] = buffer_f32(rt, to[c], so);
    }
}

// 1 / (1 + e^-s) from the hardware exp2 and reciprocal (each within about 1 ulp), given
// s2 = -log2(e) s: the kernels scale the output layer by kNegLog2e (scale_output), so the matrix
// instruction delivers s2 directly
constexpr float kNegLog2e = -1.44269504088896341f;
__device__ __forceinline__ float sigmoid_hw2(float s2) { return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(s2)); }

// the output of a pre-activation: clamp(s + 0.5) with --clamp, else the sigmoid of a pre-activation
// delivered as -log2(e) s (the output layer is scaled when !clamp)
template <class S>
__device__ __forceinline__ float out_of(float s, bool clamp) {
    return clamp ? __builtin_amdgcn_fmed3f(s + 0.5f, 0.0f, 1.0f) : sigmoid_hw2(s);
}

// Where a member's parameters come from: the weight sets of a central-difference step (kSets), or -
// in an ES step - both members' weights w0 +- sigma eps (one fused operation each, main.cpp:1852-1856)
// staged in LDS, from the block's own draw of the pair's Gaussians (NS_MLP, step, pair, k; the chunk-0
// block writes them to eps for the update: kDraw, for populations with one or two chunks per pair) or
// from the Gaussians a separate kernel drew once for all chunks (kReadEps).
enum PopFrom : int { kSets = 0, kDraw = 1, kReadEps = 2 };
struct PopSource {
    const float* wsets;                    // central differences: 2 pairs x P
    NoiseFix nt; uint64_t seed; uint32_t step; float sigma;
    const float* w0; float* eps;           // ES: the current weights and the step's Gaussians [pair][P]
};

// waves per SIMD the register allocation aims at (more would spill)
template <class S>
constexpr int pop_occupancy() { return MfmaShape<S>::kH > 32 ? 2 : (MfmaShape<S>::kIn <= 8 ? 4 : 3); }

template <class S, int Act, bool Clamp, int From>
__global__ void __launch_bounds__(64 * kPopWaves) __attribute__((amdgpu_waves_per_eu(pop_occupancy<S>()))) k_pop_mfma(DevModel m, PopSource src, int M, int Mcap,
                                                           int chunk, int chunks, const float* __restrict__ feat,
                                                           const float* __restrict__ btgt, double* __restrict__ part) {
    using Q = MfmaShape<S>;
    constexpr bool Es = From != kSets;
    __shared__ double red[kPopWaves];
    __shared__ float wpm_s[Es ? 2 * Q::kP : 1];   // ES: the + member's weights, then the - member's
    // the pixel-per-lane output layer's transposes: kOwnWave floats per wave
    __shared__ __attribute__((aligned(16))) float own_s[pop_own<S>() ? kPopWaves * kOwnWave : 4];
    // the VALU output layer's reduce-scatters: kVoTile floats per tile of a pass, per wave
    constexpr int kVoWave = kVoTile * pop_u<S>();
    __shared__ __attribute__((aligned(16))) float vo_s[valu_out<S>() && !pop_own<S>() ? kPopWaves * kVoWave : 4];
    const int lane = tid_x() & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
    const int pair = bid_x(), ch = bid_y(), sgn = wave & 1, half = wave >> 1;
    const int i16 = lane & 15, g = lane >> 4;
    constexpr int NT = pop_nt<S>();
    constexpr bool kOwn = pop_own<S>();
    constexpr bool kVOut = valu_out<S>();
    // lane byte offsets of the feature rows 4 ks + g (rows past nin are the array's zero rows) and target
    // rows out_at(g, r), or g (padding and rows past the last one read a valid row: their channel weights cw
    // are zero); the pixel-per-lane layer: target row r of pixel i16 of tile g
    uint32_t fo[Q::kKs1], to[NT];
#pragma unroll
    for (int ks = 0; ks < Q::kKs1; ks++) fo[ks] = 4u * ((uint32_t)(4 * ks + g) * (uint32_t)Mcap + (uint32_t)i16);
#pragma unroll
    for (int r = 0; r < NT; r++)
        to[r] = kOwn ? 4u * ((uint32_t)r * (uint32_t)Mcap + 32u * (uint32_t)g + (uint32_t)i16)
                     : 4u * ((uint32_t)(kVOut ? min(g, Q::kNout - 1) : max(out_at<S>(g, r), 0)) * (uint32_t)Mcap + (uint32_t)i16);
    const int s0 = ch * chunk, s1 = min(M, s0 + chunk);
    const int tiles = (s1 - s0 + 15) >> 4;
    const int mine = (tiles - half + 1) >> 1;   // this wave's tiles: 2 j + half, j < mine
    static_assert(minibatch_rows(Q::kIn) == 4 * Q::kKs1, "the feature rows the first layer's k-steps read");
    const __amdgpu_buffer_rsrc_t rf = buffer_of(feat, 4u * ((uint32_t)minibatch_rows(Q::kIn) * (uint32_t)Mcap + (uint32_t)kMinibatchSlack));
    const __amdgpu_buffer_rsrc_t rt = buffer_of(btgt, 4u * ((uint32_t)Q::kNout * (uint32_t)Mcap + (uint32_t)kMinibatchSlack));
    constexpr int U = pop_u<S>();
    // the first tiles' inputs load while the member's weights are staged
    PopTileIn<S> in0, in1;
    pop_load<S>(in0, rf, rt, 4u * (uint32_t)(s0 + 16 * half), fo, to);
    MfmaWeights<S> W;
    if constexpr (Es) {
        const uint64_t head = noise_head(src.seed, NS_MLP, src.step, (uint32_t)pair);
        float* eg = src.eps + (size_t)pair * Q::kP;
        for (int k = tid_x(); k < Q::kP; k += 64 * kPopWaves) {
            float e;
            if constexpr (From == kDraw) {
                e = gauss_at(src.nt, head, (uint64_t)k);
                if (ch == 0) eg[k] = e;
            } else {
                e = eg[k];
            }
            const float w0 = src.w0[k];
            wpm_s[k] = __builtin_fmaf(src.sigma, e, w0);
            wpm_s[Q::kP + k] = __builtin_fmaf(-src.sigma, e, w0);
        }
        __syncthreads();
        mfma_load<S>(W, wpm_s + sgn * Q::kP, lane);
    } else {
        mfma_load<S>(W, src.wsets + (size_t)(2 * pair + sgn) * Q::kP, lane);
    }
    if constexpr (!Clamp) scale_output<S>(W, kNegLog2e);
    if constexpr (Act == kActFold) scale_hidden<S>(W, fold_scale(m.leak));
    const float ak = act_k_of<Act>(m);
    // the channel weight of each of this lane's outputs (pixel-per-lane layer: output r; D layout: rows
    // 4 g + r; VALU output layer: output g), zero past the last output
    float cw[NT];
#pragma unroll
    for (int r = 0; r < NT; r++) {
        cw[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < Q::kNout; c++)
            if ((kOwn ? r : (kVOut ? g : out_at<S>(g, r))) == c) cw[r] = m.cw[c];
    }
    double e = 0.0;
    // One pass: tiles j .. j + U - 1 from c, while tiles j + U .. load into n. The loop alternates
    // two input sets, so no registers are copied between passes. The loads are issued on every pass
    // (the last one reloads its own tiles) so that the wait for them falls in the next pass.
    // whole: every tile of the pass lies inside the chunk (known at compile time: no per-lane checks)
    auto pass = [&](PopTileIn<S>& c, PopTileIn<S>& n, int j, auto whole) {
        constexpr bool kWhole = decltype(whole)::value;
        j = __builtin_amdgcn_readfirstlane(j);   // uniform: the tile arithmetic stays in SGPRs
        pop_load<S>(n, rf, rt, 4u * (uint32_t)(s0 + 16 * (2 * (j + U < mine ? j + U : j) + half)), fo, to);
        if constexpr (kOwn) {
            // the lane's own pixel (pixel i16 of tile j + g): its channel terms cw (d d), one multiply and one
            // fused multiply-add each, summed in float, then into the double
            float x[U][Q::kKsH];
            mfma_hidden<S, U, Act>(W, c.b1, ak, x);
            const f4v o = mfma_out_own<S>(W, x, own_s + wave * kOwnWave, g, i16);
            float tsum = 0.0f;
#pragma unroll
            for (int r = 0; r < NT; r++) {
                const float d = out_of<S>(o[r], Clamp) - c.t[0][r];
                tsum = __builtin_fmaf(__fmul_rn(cw[r], d), d, tsum);
            }
            if (kWhole || (j + g < mine && s0 + 16 * (2 * (j + g) + half) + i16 < s1)) e += (double)tsum;
        } else {
            // this lane's outputs' channel terms cw (d d): one multiply and one fused multiply-add each,
            // summed in float over the pass's tiles, then into the double
            float dq[pop_tt<S>()][NT], dd[pop_tt<S>()][NT];
            if constexpr (kVOut) {
                float x[U][Q::kKsH];
                mfma_hidden<S, U, Act>(W, c.b1, ak, x);
#pragma unroll
                for (int u = 0; u < U; u++) {
                    dd[u][0] = out_of<S>(valu_out_g<S>(W, x[u], vo_s + wave * kVoWave + u * kVoTile, g, i16), Clamp) - c.t[u][0];
                    dq[u][0] = __fmul_rn(cw[0], dd[u][0]);
                }
            } else {
                f4v o[U];
                mfma_forward<S, U, Act>(W, c.b1, ak, o);
#pragma unroll
                for (int u = 0; u < U; u++)
#pragma unroll
                    for (int r = 0; r < NT; r++) {
                        dd[u][r] = out_of<S>(o[u][r], Clamp) - c.t[u][r];
                        dq[u][r] = __fmul_rn(cw[r], dd[u][r]);
                    }
            }
            {
                if (kWhole || (j + U <= mine && s0 + 16 * (2 * (j + U - 1) + half) + 16 <= s1)) {   // all U tiles whole (uniform)
                    float tsum = 0.0f;
#pragma unroll
                    for (int u = 0; u < U; u++)
#pragma unroll
                        for (int r = 0; r < NT; r++) tsum = __builtin_fmaf(dq[u][r], dd[u][r], tsum);
                    e += (double)tsum;
                } else {
#pragma unroll
                    for (int u = 0; u < U; u++) {
                        const int st = s0 + 16 * (2 * (j + u) + half);   // first slot of the tile (uniform)
                        float tsum = 0.0f;
#pragma unroll
                        for (int r = 0; r < NT; r++) tsum = __builtin_fmaf(dq[u][r], dd[u][r], tsum);
                        if (j + u < mine && st + i16 < s1) e += (double)tsum;
                    }
                }
            }
        }
    };
    // this wave's tiles that lie wholly inside the chunk (tile t: slots s0 + 16 (2 t + half) + 0 .. 15)
    const int nwhole = min(mine, max(0, (s1 - s0 - 16 * half + 16) >> 5));
    int j = 0;
    for (; pop_pairs_whole<S>() && j + 2 * U <= nwhole; j += 2 * U) {   // two whole passes: one straight-line block
        pass(in0, in1, j, WholeTag<true>{});
        pass(in1, in0, j + U, WholeTag<true>{});
    }
    for (; j < mine; j += 2 * U) {
        pass(in0, in1, j, WholeTag<false>{});
        if (j + U >= mine) break;
        pass(in1, in0, j + U, WholeTag<false>{});
    }
    e = wave_sum(e);
    if (lane == 0) red[wave] = e;
    __syncthreads();
    if (tid_x() == 0) {
        part[(size_t)(2 * pair) * chunks + ch] = red[0] + red[2];
        part[(size_t)(2 * pair + 1) * chunks + ch] = red[1] + red[3];
    }
}

// ---- The ES population with the pair's first layer shared (models with one or two 16-unit hidden tiles, except the
// pixel-per-lane shapes; the launch takes it where a chunk's first-layer pre-activations stay in the L2). More than 4
// outputs: the output tile on the matrix cores, its rows packed (out_at); at most 4: valu_out_g's sums and
// reduce-scatter on the VALU, both members' output weights read from an LDS table (in registers they would cost a
// wave per SIMD). The two members of a pair differ
// in every weight by +-sigma eps, so their first layers are h+- = u +- d with u the unperturbed layer's pre-activations
// (bias + w x, the same for every pair; the minibatch launch computes it once per step, lay1[unit][slot]) and d the
// perturbation's: h- = 2 u - h+, one fused multiply-add per value instead of the - member's first-layer matrix
// instructions. A wave evaluates both members of its pair on one 16-slot tile at a time (two independent chains
// after the first layer), on tiles wave, wave + 4, ... of the chunk; the member's A operands stay in VGPRs, the
// biases come from LDS rows in operand layout (every lane of a group reads the same 16 bytes), so the two members'
// weights fit the four waves per SIMD the chains need. Every parameter is the reference's w0 +- sigma eps
// (main.cpp:1852-1856) scaled as k_pop_mfma scales it; the - member's first layer is within a few roundings of its
// own chain's, inside the 1e-5 member-loss bar.
template <class S, bool = MfmaShape<S>::kOk>
struct PopPairOk { static constexpr bool value = false; };
template <class S>
struct PopPairOk<S, true> {
    static constexpr bool value = MfmaShape<S>::kHt <= 2 && MfmaShape<S>::kH % 16 == 0 && !pop_own<S>();
};
template <class S>
constexpr bool pop_pair_ok() { return PopPairOk<S>::value; }
// bias rows per member: the first layer's kHt tiles, each deeper hidden layer's kHt, the output tile
template <class S>
constexpr int pair_bias_rows() { return MfmaShape<S>::kHt * MfmaShape<S>::kNL + 1; }
// a member's parameters in LDS, padded to whole 16-byte pieces
template <class S>
constexpr int pair_p_pad() { return (MfmaShape<S>::kP + 3) & ~3; }

// UnitCw: every channel weight is 1 (a single texture, or equally weighted ones), so cw (d d) is d d without a multiply
// Stages both members of an ES pair in LDS: wpm_s = w0 + sigma eps, then (PP floats on) w0 - sigma eps (main.cpp:1852-1856),
// scaled as k_pop_mfma scales its registers (the hidden layers by the folded activation's (1 + leak) / 2, the output
// layer by -log2 e for the hardware sigmoid); the biases also to their operand rows bias_s [member][row][4 g + r]
// (the output tile's padding rows zero), and cw_s[4 g + r] = the channel weight of output register r of lane group g.
// The Gaussians are drawn here (kDraw: the chunk-0 block writes them for the update) or read (kReadEps).
template <class S, bool Clamp, int From>
__device__ __forceinline__ void pair_stage(const DevModel& m, const PopSource& src, int pair, int ch, float* __restrict__ wpm_s,
                                           float* __restrict__ bias_s, float* __restrict__ cw_s) {
    using Q = MfmaShape<S>;
    constexpr int H = Q::kH, NIN = Q::kIn, NO = Q::kNout, RO = out_regs<S>(), NB = pair_bias_rows<S>(), PP = pair_p_pad<S>();
    constexpr int kPout = H * NIN + H + (Q::kNL - 1) * (H * H + H);   // the first output-layer parameter
    const uint64_t head = noise_head(src.seed, NS_MLP, src.step, (uint32_t)pair);
    float* eg = src.eps + (size_t)pair * Q::kP;
    const float fb = fold_scale(m.leak);
    if (tid_x() < 16) {   // the output tile's padding rows; the channel weights (zero on padding)
        const int gg = tid_x() >> 2, r = tid_x() & 3, c = out_at<S>(gg, r);
        if (c < 0) { bias_s[(NB - 1) * 16 + tid_x()] = 0.0f; bias_s[(2 * NB - 1) * 16 + tid_x()] = 0.0f; }
        cw_s[tid_x()] = c < 0 ? 0.0f : m.cw[c];
    }
    for (int k = tid_x(); k < Q::kP; k += 64 * kPopWaves) {
        float e;
        if constexpr (From == kDraw) {
            e = gauss_at(src.nt, head, (uint64_t)k);
            if (ch == 0) eg[k] = e;
        } else {
            e = eg[k];
        }
        const float w0 = src.w0[k];
        const float sc = k < kPout ? fb : (Clamp ? 1.0f : kNegLog2e);
        const float vp = __builtin_fmaf(src.sigma, e, w0) * sc, vm = __builtin_fmaf(-src.sigma, e, w0) * sc;
        wpm_s[k] = vp;
        wpm_s[PP + k] = vm;
        int row = -1, col = 0;   // a bias: its operand row and column
        if (k >= H * NIN && k < H * NIN + H) {
            row = (k - H * NIN) >> 4; col = (k - H * NIN) & 15;
        } else if (k >= H * NIN + H && k < kPout) {
            const int q = k - (H * NIN + H), l = q / (H * H + H), o = q - l * (H * H + H) - H * H;
            if (o >= 0) { row = Q::kHt * (1 + l) + (o >> 4); col = o & 15; }
        } else if (k >= kPout + NO * H) {
            const int c = k - (kPout + NO * H);
            row = NB - 1; col = 4 * (c / RO) + c % RO;   // output c sits in register c % RO of lane group c / RO
        }
        if (row >= 0) { bias_s[row * 16 + col] = vp; bias_s[(NB + row) * 16 + col] = vm; }
    }
}

template <class S, bool Clamp, int From, bool UnitCw>
__global__ void __launch_bounds__(64 * kPopWaves) __attribute__((amdgpu_waves_per_eu(pop_occupancy<S>()))) k_pop_pair(DevModel m, PopSource src, int M, int Mcap,
                                                            int chunk, int chunks, const float* __restrict__ feat,
                                                            const float* __restrict__ btgt, const float* __restrict__ lay1,
                                                            double* __restrict__ part) {
    using Q = MfmaShape<S>;
    static_assert(From != kSets && pop_pair_ok<S>(), "an ES step of a shape the pair kernel takes");
    constexpr int H = Q::kH, NIN = Q::kIn, NO = Q::kNout, RO = out_regs<S>(), NB = pair_bias_rows<S>(), PP = pair_p_pad<S>();
    constexpr int kPout = H * NIN + H + (Q::kNL - 1) * (H * H + H);   // the first output-layer parameter
    __shared__ double red[2][kPopWaves];
    __shared__ __attribute__((aligned(16))) float wpm_s[2 * PP];          // the + member's parameters, then the - member's
    __shared__ __attribute__((aligned(16))) float bias_s[2 * NB * 16];    // [member][row][4 g + r]
    __shared__ __attribute__((aligned(16))) float cw_s[16];               // the channel weight of register r of group g
    // at most 4 outputs: the output layer on the VALU (valu_out_g's sums and reduce-scatter), its weights from LDS:
    // [member][lane group][bias, then k-step 0 .. kKsH - 1][output 0 .. 3], and each wave's two reduce-scatter tiles
    constexpr bool kVOut = valu_out<S>();
    constexpr int kWo = kVOut ? 2 * 4 * (Q::kKsH + 1) * 4 : 4;
    __shared__ __attribute__((aligned(16))) float wo_s[kWo];
    __shared__ __attribute__((aligned(16))) float vo_s[kVOut ? kPopWaves * 2 * kVoTile : 4];
    const int lane = tid_x() & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
    const int pair = bid_x(), ch = bid_y();
    const int i16 = lane & 15, g = lane >> 4;
    const int s0 = ch * chunk, s1 = min(M, s0 + chunk);
    const int tiles = (s1 - s0 + 15) >> 4;
    const int mine = (tiles - wave + kPopWaves - 1) / kPopWaves;   // this wave's tiles: wave + 4 j, j < mine
    // lane byte offsets: feature rows 4 ks + g, first-layer rows 16 ot + 4 g + r, target rows out_at(g, r) (a valid row
    // for padding: its channel weight is zero)
    // (register r of lane group g holds output RO g + r, so row r of a group is its first row + r)
    static_assert(out_at<S>(3, RO - 1) == 3 * RO + RO - 1 || out_at<S>(3, RO - 1) < 0, "packed output rows");
    const uint32_t fo = 4u * ((uint32_t)g * (uint32_t)Mcap + (uint32_t)i16);
    const uint32_t uo = 4u * (4u * (uint32_t)g * (uint32_t)Mcap + (uint32_t)i16);
    const uint32_t to = 4u * ((uint32_t)min(RO * g, NO - RO) * (uint32_t)Mcap + (uint32_t)i16);
    const __amdgpu_buffer_rsrc_t rf = buffer_of(feat, 4u * ((uint32_t)minibatch_rows(NIN) * (uint32_t)Mcap + (uint32_t)kMinibatchSlack));
    const __amdgpu_buffer_rsrc_t rt = buffer_of(btgt, 4u * ((uint32_t)NO * (uint32_t)Mcap + (uint32_t)kMinibatchSlack));
    const __amdgpu_buffer_rsrc_t ru = buffer_of(lay1, 4u * ((uint32_t)H * (uint32_t)Mcap + (uint32_t)kMinibatchSlack));
    // a tile's inputs, loaded one pass ahead; its targets at the start of its own pass (used at the end)
    struct TileIn { float b1[Q::kKs1]; float u[Q::kHt][4]; };
    auto tile_off = [&](int j) {   // tile wave + 4 j (uniform)
        return (uint32_t)__builtin_amdgcn_readfirstlane((int)(4u * (uint32_t)(s0 + 16 * (wave + kPopWaves * j))));
    };
    auto load = [&](TileIn& in, int j) {
        const uint32_t so = tile_off(j);
#pragma unroll
        for (int ks = 0; ks < Q::kKs1; ks++) in.b1[ks] = buffer_f32(rf, fo, so + 16u * (uint32_t)ks * (uint32_t)Mcap);
#pragma unroll
        for (int ot = 0; ot < Q::kHt; ot++)
#pragma unroll
            for (int r = 0; r < 4; r++) in.u[ot][r] = buffer_f32(ru, uo, so + 4u * (uint32_t)(16 * ot + r) * (uint32_t)Mcap);
    };
    TileIn in0, in1;
    load(in0, 0);
    pair_stage<S, Clamp, From>(m, src, pair, ch, wpm_s, bias_s, cw_s);
    __syncthreads();
    if constexpr (kVOut) {   // the output layer's table from the staged (scaled) parameters
        for (int i = tid_x(); i < kWo; i += 64 * kPopWaves) {
            const int c = i & 3, ks = (i >> 2) % (Q::kKsH + 1) - 1, gg = (i >> 2) / (Q::kKsH + 1) % 4, mem = i / (4 * (Q::kKsH + 1) * 4);
            const float* wm = wpm_s + mem * PP + kPout;
            float v = 0.0f;
            if (c < NO) {
                if (ks < 0) v = gg == 0 ? wm[NO * H + c] : 0.0f;   // the bias, in lane group 0 (valu_out_g's W.bo)
                else if (hidden_input<Q>(ks, gg) < H) v = wm[c * H + hidden_input<Q>(ks, gg)];
            }
            wo_s[i] = v;
        }
        __syncthreads();
    }
    MfmaWeights<S> Wp, Wm;   // the A operands of both members (their bias fields unused)
    mfma_load<S>(Wp, wpm_s, lane);
    mfma_load<S>(Wm, wpm_s + PP, lane);
    const float ak = act_k_of<kActFold>(m);
    auto bias = [&](int mem, int row) { return *reinterpret_cast<const f4v*>(bias_s + (mem * NB + row) * 16 + 4 * g); };
    // valu_out_g of member mem with its weights from wo_s: output g of pixel i16 in lane (g, i16), zero past nout
    auto vout = [&](int mem, const float (&x)[Q::kKsH]) {
        const float* wg = wo_s + (mem * 4 + g) * (Q::kKsH + 1) * 4;
        float* t = vo_s + (wave * 2 + mem) * kVoTile;
        f4v p = *reinterpret_cast<const f4v*>(wg);
#pragma unroll
        for (int ks = 0; ks < Q::kKsH; ks++) {
            const f4v wv = *reinterpret_cast<const f4v*>(wg + 4 * (ks + 1));
#pragma unroll
            for (int c = 0; c < NO; c++) p[c] = __builtin_fmaf(wv[c], x[ks], p[c]);
        }
#pragma unroll
        for (int c = 0; c < 4; c++) t[i16 * kOwnRow + 4 * c + g] = p[c];
        wave_lds_fence();
        const f4v v = *reinterpret_cast<const f4v*>(t + i16 * kOwnRow + 4 * g);
        wave_lds_fence();
        return (v[0] + v[2]) + (v[1] + v[3]);
    };
    double ep = 0.0, em = 0.0;
    float fp = 0.0f, fm = 0.0f;   // the float sums of this lane's terms over the passes since the last double add
    auto pass = [&](TileIn& c, TileIn& n, int j) {
        j = __builtin_amdgcn_readfirstlane(j);
        float tt[RO];
        {
            const uint32_t so = tile_off(j);
#pragma unroll
            for (int r = 0; r < RO; r++) tt[r] = buffer_f32(rt, to, so + 4u * (uint32_t)r * (uint32_t)Mcap);
        }
        load(n, j + 1 < mine ? j + 1 : j);
        // first layer: the + member's chain, the - member as 2 u - h+
        f4v hp[Q::kHt], hm[Q::kHt];
#pragma unroll
        for (int ot = 0; ot < Q::kHt; ot++) hp[ot] = bias(0, ot);
#pragma unroll
        for (int ks = 0; ks < Q::kKs1; ks++)
#pragma unroll
            for (int ot = 0; ot < Q::kHt; ot++) hp[ot] = mfma4(Wp.a1[ot][ks], c.b1[ks], hp[ot]);
#pragma unroll
        for (int ot = 0; ot < Q::kHt; ot++)
#pragma unroll
            for (int r = 0; r < 4; r++) hm[ot][r] = __builtin_fmaf(2.0f, c.u[ot][r], -hp[ot][r]);
        float xp[Q::kKsH], xm[Q::kKsH];
#pragma unroll
        for (int ot = 0; ot < Q::kHt; ot++)
#pragma unroll
            for (int r = 0; r < 4; r++) { xp[4 * ot + r] = act<kActFold>(hp[ot][r], ak); xm[4 * ot + r] = act<kActFold>(hm[ot][r], ak); }
#pragma unroll
        for (int l = 0; l < Q::kNL - 1; l++) {
            f4v ap[Q::kHt], am[Q::kHt];
#pragma unroll
            for (int ot = 0; ot < Q::kHt; ot++) { ap[ot] = bias(0, Q::kHt * (1 + l) + ot); am[ot] = bias(1, Q::kHt * (1 + l) + ot); }
#pragma unroll
            for (int ks = 0; ks < Q::kKsH; ks++)
#pragma unroll
                for (int ot = 0; ot < Q::kHt; ot++) {
                    ap[ot] = mfma4(Wp.ah[l][ot][ks], xp[ks], ap[ot]);
                    am[ot] = mfma4(Wm.ah[l][ot][ks], xm[ks], am[ot]);
                }
#pragma unroll
            for (int ot = 0; ot < Q::kHt; ot++)
#pragma unroll
                for (int r = 0; r < 4; r++) { xp[4 * ot + r] = act<kActFold>(ap[ot][r], ak); xm[4 * ot + r] = act<kActFold>(am[ot][r], ak); }
        }
        f4v op, om;
        if constexpr (kVOut) {
            op[0] = vout(0, xp);
            om[0] = vout(1, xm);
        } else {
            op = bias(0, NB - 1);
            om = bias(1, NB - 1);
#pragma unroll
            for (int ks = 0; ks < Q::kKsH; ks++) {
                op = mfma4(Wp.ao[ks], xp[ks], op);
                om = mfma4(Wm.ao[ks], xm[ks], om);
            }
        }
        // each member's channel terms cw (d d) (a multiply, unless every cw is 1, and a fused multiply-add each), summed
        // in float over this lane's outputs of the tile and over the loop's two passes, then into the member's double
        float tp = 0.0f, tm = 0.0f;
        const f4v cw = *reinterpret_cast<const f4v*>(cw_s + 4 * g);
        constexpr bool kUnit = UnitCw && NO == 4 * RO;   // (with padding rows their zero weight is still needed)
#pragma unroll
        for (int r = 0; r < RO; r++) {
            const float dp = out_of<S>(op[r], Clamp) - tt[r], dm = out_of<S>(om[r], Clamp) - tt[r];
            tp = __builtin_fmaf(kUnit ? dp : __fmul_rn(cw[r], dp), dp, tp);
            tm = __builtin_fmaf(kUnit ? dm : __fmul_rn(cw[r], dm), dm, tm);
        }
        if (s0 + 16 * (wave + kPopWaves * j) + i16 < s1) { fp += tp; fm += tm; }
    };
    for (int j = 0; j < mine; j += 2) {
        pass(in0, in1, j);
        if (j + 1 < mine) pass(in1, in0, j + 1);
        ep += (double)fp; em += (double)fm;
        fp = 0.0f; fm = 0.0f;
    }
    ep = wave_sum(ep);
    em = wave_sum(em);
    if (lane == 0) { red[0][wave] = ep; red[1][wave] = em; }
    __syncthreads();
    if (tid_x() == 0) {
        part[(size_t)(2 * pair) * chunks + ch] = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
        part[(size_t)(2 * pair + 1) * chunks + ch] = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    }
}

// ---- The pair population kernel of the pixel-per-lane shapes (at most 4 outputs, one 16-unit hidden tile: rgb256's
// 6-16-16-3). As k_pop_pair, both members of the pair in each wave and the - member's first layer as 2 u - h+; a pass
// takes two of the wave's tiles, so four chains run after the first layer. The output layer's exchange (mfma_out_own)
// takes the + member's two tiles as its tiles 0 and 1 and the - member's as 2 and 3, and each lane's 4x4x1 A operands
// are the output weights of the member its lane group holds: lane (g, j) ends with the outputs of pixel j of the pass's
// tile g & 1 for member g >> 1, and adds that pixel's channel terms to its member's sum.
template <class S, bool = MfmaShape<S>::kOk>
struct PopPairOwnOk { static constexpr bool value = false; };
template <class S>
struct PopPairOwnOk<S, true> { static constexpr bool value = pop_own<S>() && MfmaShape<S>::kH == 16; };
template <class S>
constexpr bool pop_pair_own_ok() { return PopPairOwnOk<S>::value; }

template <class S, bool Clamp, int From, bool UnitCw>
__global__ void __launch_bounds__(64 * kPopWaves) __attribute__((amdgpu_waves_per_eu(pop_occupancy<S>()))) k_pop_pair_own(
        DevModel m, PopSource src, int M, int Mcap, int chunk, int chunks, const float* __restrict__ feat, const float* __restrict__ btgt,
        const float* __restrict__ lay1, double* __restrict__ part) {
    using Q = MfmaShape<S>;
    static_assert(From != kSets && pop_pair_own_ok<S>() && Q::kHt == 1, "an ES step of a pixel-per-lane shape");
    constexpr int H = Q::kH, NIN = Q::kIn, NO = Q::kNout, NB = pair_bias_rows<S>(), PP = pair_p_pad<S>();
    __shared__ double red[2][kPopWaves];
    __shared__ __attribute__((aligned(16))) float wpm_s[2 * PP];          // the + member's parameters, then the - member's
    __shared__ __attribute__((aligned(16))) float bias_s[2 * NB * 16];    // [member][row][4 g + r]
    __shared__ __attribute__((aligned(16))) float cw_s[16];
    __shared__ __attribute__((aligned(16))) float own_s[kPopWaves * kOwnWave];   // each wave's output-layer exchange
    const int lane = tid_x() & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
    const int pair = bid_x(), ch = bid_y();
    const int i16 = lane & 15, g = lane >> 4;
    const int s0 = ch * chunk, s1 = min(M, s0 + chunk);
    const int tiles = (s1 - s0 + 15) >> 4;
    const int mine = (tiles - wave + kPopWaves - 1) / kPopWaves;   // this wave's tiles: wave + 4 q, q < mine
    // lane byte offsets: feature rows 4 ks + g, first-layer rows 4 g + r, and the targets of pixel i16 of the pass's tile
    // g & 1 (64 slots after its tile 0)
    const uint32_t fo = 4u * ((uint32_t)g * (uint32_t)Mcap + (uint32_t)i16);
    const uint32_t uo = 4u * (4u * (uint32_t)g * (uint32_t)Mcap + (uint32_t)i16);
    const uint32_t to = 4u * ((uint32_t)i16 + 64u * (uint32_t)(g & 1));
    const __amdgpu_buffer_rsrc_t rf = buffer_of(feat, 4u * ((uint32_t)minibatch_rows(NIN) * (uint32_t)Mcap + (uint32_t)kMinibatchSlack));
    const __amdgpu_buffer_rsrc_t rt = buffer_of(btgt, 4u * ((uint32_t)NO * (uint32_t)Mcap + (uint32_t)kMinibatchSlack));
    const __amdgpu_buffer_rsrc_t ru = buffer_of(lay1, 4u * ((uint32_t)H * (uint32_t)Mcap + (uint32_t)kMinibatchSlack));
    // the inputs of a pass's two tiles, loaded one pass ahead; the targets at the start of their own pass
    struct TileIn { float b1[2][Q::kKs1]; float u[2][4]; };
    auto tile_off = [&](int q) {   // tile wave + 4 q (uniform)
        return (uint32_t)__builtin_amdgcn_readfirstlane((int)(4u * (uint32_t)(s0 + 16 * (wave + kPopWaves * q))));
    };
    auto load = [&](TileIn& in, int j) {   // tiles 2 j and 2 j + 1 (a tile past the wave's last reads its last)
#pragma unroll
        for (int v = 0; v < 2; v++) {
            const uint32_t so = tile_off(min(2 * j + v, mine - 1));
#pragma unroll
            for (int ks = 0; ks < Q::kKs1; ks++) in.b1[v][ks] = buffer_f32(rf, fo, so + 16u * (uint32_t)ks * (uint32_t)Mcap);
#pragma unroll
            for (int r = 0; r < 4; r++) in.u[v][r] = buffer_f32(ru, uo, so + 4u * (uint32_t)r * (uint32_t)Mcap);
        }
    };
    TileIn in0, in1;
    if (mine > 0) load(in0, 0);
    pair_stage<S, Clamp, From>(m, src, pair, ch, wpm_s, bias_s, cw_s);
    __syncthreads();
    MfmaWeights<S> Wp, Wm, Wo;   // the A operands of both members; the output layer of the member of this lane group
    mfma_load<S>(Wp, wpm_s, lane);
    mfma_load<S>(Wm, wpm_s + PP, lane);
    mfma_load<S>(Wo, wpm_s + (g >> 1) * PP, lane);
    const float ak = act_k_of<kActFold>(m);
    auto bias = [&](int mem, int row) { return *reinterpret_cast<const f4v*>(bias_s + (mem * NB + row) * 16 + 4 * g); };
    float cw[NO];
#pragma unroll
    for (int r = 0; r < NO; r++) cw[r] = m.cw[r];
    double e = 0.0;   // this lane's member's sum
    auto pass = [&](TileIn& c, TileIn& n, int j) {
        j = __builtin_amdgcn_readfirstlane(j);
        float tt[NO];
        {
            const uint32_t so = tile_off(2 * j);
#pragma unroll
            for (int r = 0; r < NO; r++) tt[r] = buffer_f32(rt, to, so + 4u * (uint32_t)r * (uint32_t)Mcap);
        }
        load(n, 2 * j + 2 < mine ? j + 1 : j);
        float x[4][Q::kKsH];   // the last hidden layer: + member's tiles 0, 1, then the - member's
#pragma unroll
        for (int v = 0; v < 2; v++) {
            f4v hp = bias(0, 0), hm;
#pragma unroll
            for (int ks = 0; ks < Q::kKs1; ks++) hp = mfma4(Wp.a1[0][ks], c.b1[v][ks], hp);
#pragma unroll
            for (int r = 0; r < 4; r++) hm[r] = __builtin_fmaf(2.0f, c.u[v][r], -hp[r]);
#pragma unroll
            for (int r = 0; r < 4; r++) { x[v][r] = act<kActFold>(hp[r], ak); x[2 + v][r] = act<kActFold>(hm[r], ak); }
        }
#pragma unroll
        for (int l = 0; l < Q::kNL - 1; l++) {
            f4v a[4];
#pragma unroll
            for (int t = 0; t < 4; t++) a[t] = bias(t >> 1, 1 + l);
#pragma unroll
            for (int ks = 0; ks < Q::kKsH; ks++)
#pragma unroll
                for (int t = 0; t < 4; t++) a[t] = mfma4(t < 2 ? Wp.ah[l][0][ks] : Wm.ah[l][0][ks], x[t][ks], a[t]);
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) x[t][r] = act<kActFold>(a[t][r], ak);
        }
        const f4v o = mfma_out_own<S>(Wo, x, own_s + wave * kOwnWave, g, i16);
        // the lane's pixel: its channel terms cw (d d) (a multiply, unless every cw is 1, and a fused multiply-add each)
        float tsum = 0.0f;
#pragma unroll
        for (int r = 0; r < NO; r++) {
            const float d = out_of<S>(o[r], Clamp) - tt[r];
            tsum = __builtin_fmaf(UnitCw ? d : __fmul_rn(cw[r], d), d, tsum);
        }
        const int q = 2 * j + (g & 1);
        if (q < mine && s0 + 16 * (wave + kPopWaves * q) + i16 < s1) e += (double)tsum;
    };
    for (int j = 0; 2 * j < mine; j += 2) {
        pass(in0, in1, j);
        if (2 * j + 2 < mine) pass(in1, in0, j + 1);
    }
    const double ep = wave_sum(g < 2 ? e : 0.0), em = wave_sum(g < 2 ? 0.0 : e);
    if (lane == 0) { red[0][wave] = ep; red[1][wave] = em; }
    __syncthreads();
    if (tid_x() == 0) {
        part[(size_t)(2 * pair) * chunks + ch] = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
        part[(size_t)(2 * pair + 1) * chunks + ch] = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    }
}

// The latent pair evaluation (LatentTrainer::step_impl, main.cpp:1990-2007) on the matrix cores:
// block (512 or 256 pixels, pair k), each wave a quarter of them in rounds of 64. In a round every
// lane builds the features of its own pixel with the pair's texels perturbed by +sg eps and by
// -sg eps (features_pm: both members from one set of taps and texel loads), and an exchange through
// the wave's own LDS rows (tiles_of) turns the 64 pixels into the B operands of four 16-pixel tiles:
// no barrier, so a wave's feature loads overlap other waves' matrix work. Each
// tile's + and - members are evaluated together; a pixel's error is decode_err's float sum of
// cw (d d) over its channels (a lane's out_regs in ascending order, then the lane groups pairwise: within
// a few ulp of the reference's ascending chain), and dpix = (e+ - e-) * inv_px.
// rounds of 64 pixels per wave, at most: 2 (512 pixels per block), or 1 for wide inputs; the launch may
// take fewer (`rounds`) to spread a small image over more blocks. One rule for the kernel and its
// launchers (the host checks a launch's rounds against it: the kernel stops at this count).
__host__ __device__ constexpr int lat_rounds_of(int nin) { return nin <= 8 ? 2 : 1; }
template <class S>
constexpr int lat_rounds() { return lat_rounds_of(MfmaShape<S>::kIn); }

// The features of one pixel for both members of a latent pair at once (fixed shapes): every tap and texel
// load is shared, each member's texel value is its own fused zb +- sg eps (a level outside `mask` is
// unperturbed), and each member's blend is the single-member blend - so fp and fm equal features<S> with
// PerturbedLatent{ z, eps, sg, mask } and { z, eps, -sg, mask }. Texels are read through raw buffers with
// 32-bit byte offsets (a latent holds fewer than 2^30 floats). The code has no branch per texel: a level
// outside `mask` reads its Gaussians through an empty buffer (rn: every load returns 0 without touching
// memory), so fma(+-sg, 0, zb) = zb, up to the sign of a zero texel, which no output can see (the layers'
// sums and the activation treat +0 and -0 alike). A branch per texel (or stores under a branch) makes the
// compiler keep the features in scratch.
template <int C>
__device__ __forceinline__ void sample_level_pm(const DevLevel& L, __amdgpu_buffer_rsrc_t rz, __amdgpu_buffer_rsrc_t re,
                                                float sg, const Tap& t, float* fp, float* fm) {
    const uint32_t off = (uint32_t)L.off, LW = (uint32_t)L.W, LC = (uint32_t)L.C;
    const uint32_t a = 4u * (off + ((uint32_t)t.y0 * LW + (uint32_t)t.x0) * LC);
    if (L.nearest) {
#pragma unroll
        for (int c = 0; c < C; c++) {
            const float zb = buffer_f32(rz, a + 4u * c, 0u), ee = buffer_f32(re, a + 4u * c, 0u);
            fp[c] = __builtin_fmaf(sg, ee, zb);
            fm[c] = __builtin_fmaf(-sg, ee, zb);
        }
        return;
    }
    const uint32_t tap[4] = { a, 4u * (off + ((uint32_t)t.y0 * LW + (uint32_t)t.x1) * LC),
                              4u * (off + ((uint32_t)t.y1 * LW + (uint32_t)t.x0) * LC),
                              4u * (off + ((uint32_t)t.y1 * LW + (uint32_t)t.x1) * LC) };
    const Blend w = blend_of(t);
#pragma unroll
    for (int c = 0; c < C; c++) {
        float vp[4], vm[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float zb = buffer_f32(rz, tap[q] + 4u * c, 0u), ee = buffer_f32(re, tap[q] + 4u * c, 0u);
            vp[q] = __builtin_fmaf(sg, ee, zb);
            vm[q] = __builtin_fmaf(-sg, ee, zb);
        }
        fp[c] = blend(w, vp[0], vp[1], vp[2], vp[3]);
        fm[c] = blend(w, vm[0], vm[1], vm[2], vm[3]);
    }
}

template <class S>
__device__ __forceinline__ void features_pm(const DevModel& m, __amdgpu_buffer_rsrc_t rz, __amdgpu_buffer_rsrc_t re, __amdgpu_buffer_rsrc_t rn,
                                            float sg, unsigned mask,
                                            int px, int py, float (&fp)[S::kMaxIn], float (&fm)[S::kMaxIn]) {
    static_assert(S::kFixed, "fixed shapes only");
    const float u = pixel_u(px, m.W), v = pixel_u(py, m.H);
    const Tap t0 = tap_of(m.lv[0].W, m.lv[0].H, m.lv[0].nearest != 0, u, v);
    Tap t1 = t0;
    sample_level_pm<S::kC0>(m.lv[0], rz, (mask & 1u) ? re : rn, sg, t0, fp, fm);
    if constexpr (S::kC1 > 0) {
        t1 = tap_of(m.lv[1].W, m.lv[1].H, m.lv[1].nearest != 0, u, v);
        sample_level_pm<S::kC1>(m.lv[1], rz, ((mask >> 1) & 1u) ? re : rn, sg, t1, fp + S::kC0, fm + S::kC0);
    }
    if constexpr (S::kC2 > 0) {
        const Tap t2 = tap_of(m.lv[2].W, m.lv[2].H, m.lv[2].nearest != 0, u, v);
        sample_level_pm<S::kC2>(m.lv[2], rz, ((mask >> 2) & 1u) ? re : rn, sg, t2, fp + S::kC0 + S::kC1, fm + S::kC0 + S::kC1);
    }
    constexpr int k0 = S::kC0 + S::kC1 + S::kC2;
#pragma unroll
    for (int q = 0; q < S::kNpos; q++) {
        const bool uv = m.pos[q] == 0;
        fp[k0 + 2 * q] = fm[k0 + 2 * q] = __builtin_fmaf(uv ? u : t1.fx, 2.0f, -1.0f);
        fp[k0 + 2 * q + 1] = fm[k0 + 2 * q + 1] = __builtin_fmaf(uv ? v : t1.fy, 2.0f, -1.0f);
    }
}

// Models whose latent step perturbs level 1 only (level 0 searched under --qat, so the step's mask is 2) and whose
// level-0 channels and positional features fill whole k-steps of the first layer: the latent pair takes those
// inputs first (level 0, then the positional features, then level 1), so the k-steps over them are one chain of
// matrix instructions for both members of a pair, which each member's level-1 k-steps continue. Each unit's
// first-layer sum then adds the same products in that order instead of the reference's (main.cpp:603-627).
// The shared k-steps, or 0 where the layout has none.
template <class S>
constexpr int lat_shared_ksteps() {
    return (S::kFixed && S::kC2 == 0 && S::kC1 > 0 && (S::kC0 + 2 * S::kNpos) % 4 == 0) ? (S::kC0 + 2 * S::kNpos) / 4 : 0;
}
// position p of that order holds input map(p) of the reference's order
template <class S>
struct InLatShared {
    __host__ __device__ static constexpr int map(int p) {
        return p < S::kC0 ? p : (p < S::kC0 + 2 * S::kNpos ? S::kC0 + S::kC1 + (p - S::kC0) : S::kC0 + (p - S::kC0 - 2 * S::kNpos));
    }
};
template <bool B, class A, class C> struct PickType { using type = A; };
template <class A, class C> struct PickType<false, A, C> { using type = C; };

// sample_latent of an unperturbed level through its raw buffer (sample_level_pm's loads and blend, one member)
template <int C>
__device__ __forceinline__ void sample_level_plain(const DevLevel& L, __amdgpu_buffer_rsrc_t rz, const Tap& t, float* f) {
    const uint32_t off = (uint32_t)L.off, LW = (uint32_t)L.W, LC = (uint32_t)L.C;
    const uint32_t a = 4u * (off + ((uint32_t)t.y0 * LW + (uint32_t)t.x0) * LC);
    if (L.nearest) {
#pragma unroll
        for (int c = 0; c < C; c++) f[c] = buffer_f32(rz, a + 4u * c, 0u);
        return;
    }
    const uint32_t tap[4] = { a, 4u * (off + ((uint32_t)t.y0 * LW + (uint32_t)t.x1) * LC),
                              4u * (off + ((uint32_t)t.y1 * LW + (uint32_t)t.x0) * LC),
                              4u * (off + ((uint32_t)t.y1 * LW + (uint32_t)t.x1) * LC) };
    const Blend w = blend_of(t);
#pragma unroll
    for (int c = 0; c < C; c++)
        f[c] = blend(w, buffer_f32(rz, tap[0] + 4u * c, 0u), buffer_f32(rz, tap[1] + 4u * c, 0u), buffer_f32(rz, tap[2] + 4u * c, 0u),
                     buffer_f32(rz, tap[3] + 4u * c, 0u));
}

// The features of one pixel for a latent pair in the shared order (lat_shared_ksteps): fs = level 0 and the
// positional features, common to both members; fp / fm = level 1 perturbed by +sg eps / -sg eps (features_pm's
// values, in another arrangement).
template <class S>
__device__ __forceinline__ void features_lat_shared(const DevModel& m, __amdgpu_buffer_rsrc_t rz, __amdgpu_buffer_rsrc_t re, float sg,
                                                    int px, int py, float (&fs)[S::kC0 + 2 * S::kNpos], float (&fp)[S::kC1],
                                                    float (&fm)[S::kC1]) {
    const float u = pixel_u(px, m.W), v = pixel_u(py, m.H);
    const Tap t0 = tap_of(m.lv[0].W, m.lv[0].H, m.lv[0].nearest != 0, u, v);
    const Tap t1 = tap_of(m.lv[1].W, m.lv[1].H, m.lv[1].nearest != 0, u, v);
    sample_level_plain<S::kC0>(m.lv[0], rz, t0, fs);
    sample_level_pm<S::kC1>(m.lv[1], rz, re, sg, t1, fp, fm);
#pragma unroll
    for (int q = 0; q < S::kNpos; q++) {
        const bool uv = m.pos[q] == 0;
        fs[S::kC0 + 2 * q] = __builtin_fmaf(uv ? u : t1.fx, 2.0f, -1.0f);
        fs[S::kC0 + 2 * q + 1] = __builtin_fmaf(uv ? v : t1.fy, 2.0f, -1.0f);
    }
}

// The column and row of pixel base + lane for a wave's 64 pixels from base (a multiple of 64): when the
// image's width is a multiple of 64 they share one row (a scalar division), else each lane divides (pixels
// past the last clamped to it).
__device__ __forceinline__ void round_pixel(const DevModel& m, int base, int lane, int& px, int& py) {
    if (m.W % 64 == 0 && base < m.npix) {
        const int row = base / m.W;
        px = base - row * m.W + lane;
        py = row;
    } else {
        const int pr = min(base + lane, m.npix - 1);
        px = pr % m.W;
        py = pr / m.W;
    }
}


// One 16-pixel tile of a latent pair: both members' MLPs on the tile's first-layer operands (Sh > 0: the shared
// k-steps' bs, continued by each member's own bp / bm; Sh = 0: each member's whole first layer bp / bm), each lane's
// channel terms cw (d d) (its out_regs in ascending order, or its one on the VALU output layer), the pixel's four
// lane groups added pairwise for each member (group_sums), and (e+ - e-) inv_px written to out[p] by lane group 0.
template <class S, int Act, bool Clamp, int Sh, bool UnitCw>
__device__ __forceinline__ void lat_pair_tile(const DevModel& m, const MfmaWeights<S>& W, float ak, const float (&cw)[4],
                                              const float (&bs)[Sh > 0 ? Sh : 1],
                                              const float (&bp)[Sh > 0 ? MfmaShape<S>::kKs1 - Sh : MfmaShape<S>::kKs1],
                                              const float (&bm)[Sh > 0 ? MfmaShape<S>::kKs1 - Sh : MfmaShape<S>::kKs1],
                                              const float (&tt)[4], float* vo, float* sums, int g, int i16, int p,
                                              float* __restrict__ out) {
    using Q = MfmaShape<S>;
    constexpr int NO = Q::kNout, kM = Q::kKs1 - Sh;
    constexpr bool kVOut = valu_out<S>();
    // the first layer's pre-activations of both members (D layout)
    f4v a1[2][Q::kHt];
    if constexpr (Sh > 0) {
        f4v as[Q::kHt];
#pragma unroll
        for (int ot = 0; ot < Q::kHt; ot++) as[ot] = W.c1[ot];
#pragma unroll
        for (int ks = 0; ks < Sh; ks++)
#pragma unroll
            for (int ot = 0; ot < Q::kHt; ot++) as[ot] = mfma4(W.a1[ot][ks], bs[ks], as[ot]);
#pragma unroll
        for (int ot = 0; ot < Q::kHt; ot++) { a1[0][ot] = as[ot]; a1[1][ot] = as[ot]; }
#pragma unroll
        for (int ks = 0; ks < kM; ks++)
#pragma unroll
            for (int v = 0; v < 2; v++)
#pragma unroll
                for (int ot = 0; ot < Q::kHt; ot++) a1[v][ot] = mfma4(W.a1[ot][Sh + ks], v ? bm[ks] : bp[ks], a1[v][ot]);
    } else {
        float b1[2][Q::kKs1];
#pragma unroll
        for (int ks = 0; ks < Q::kKs1; ks++) { b1[0][ks] = bp[ks]; b1[1][ks] = bm[ks]; }
        mfma_layer1<S, 2>(W, b1, a1);
    }
    float ep = 0.0f, em = 0.0f;
    if constexpr (kVOut) {
        float x[2][Q::kKsH];
        mfma_hidden_from1<S, 2, Act>(W, a1, ak, x);
        const float dp = out_of<S>(valu_out_g<S>(W, x[0], vo, g, i16), Clamp) - tt[0],
                    dm = out_of<S>(valu_out_g<S>(W, x[1], vo + kVoTile, g, i16), Clamp) - tt[0];
        constexpr bool kUnit = UnitCw && NO == 4;   // (lane groups past nout need their zero weight)
        ep = kUnit ? __fmul_rn(dp, dp) : __fmul_rn(cw[0], __fmul_rn(dp, dp));
        em = kUnit ? __fmul_rn(dm, dm) : __fmul_rn(cw[0], __fmul_rn(dm, dm));
    } else {
        float x[2][Q::kKsH];
        mfma_hidden_from1<S, 2, Act>(W, a1, ak, x);
        f4v o[2];
        mfma_output<S, 2>(W, x, o);
#pragma unroll
        for (int r = 0; r < out_regs<S>(); r++) {
            const float dp = out_of<S>(o[0][r], Clamp) - tt[r], dm = out_of<S>(o[1][r], Clamp) - tt[r];
            constexpr bool kUnit = UnitCw && NO == 4 * out_regs<S>();   // (padding rows need their zero weight)
            ep = kUnit ? __builtin_fmaf(dp, dp, ep) : __builtin_fmaf(cw[r], __fmul_rn(dp, dp), ep);
            em = kUnit ? __builtin_fmaf(dm, dm, em) : __builtin_fmaf(cw[r], __fmul_rn(dm, dm), em);
        }
    }
    float sp, sm;
    group_sums(ep, em, sums, g, i16, sp, sm);
    if (g == 0 && p < m.npix) out[p] = __fmul_rn(sp - sm, m.inv_px);
}

// Sh > 0: the shared first-layer k-steps of lat_shared_ksteps (the launch's mask must be 2: level 1 perturbed only).
// UnitCw: every channel weight is 1, so a pixel's error terms are d d (fused into the sum where a lane holds several)
template <class S, int Act, bool Clamp, int Sh = 0, bool UnitCw = false>
__global__ void __launch_bounds__(256) k_lat_pair_mfma(DevModel m, const float* __restrict__ w, const float* __restrict__ zdec,
                                                      const float* __restrict__ eps, const float* __restrict__ tgt, float sg,
                                                      unsigned mask, float* __restrict__ dpix, int rounds) {
    using Q = MfmaShape<S>;
    constexpr int NO = Q::kNout, kRounds = lat_rounds<S>();
    static_assert(Sh == 0 || Sh == lat_shared_ksteps<S>(), "the shared k-steps of the layout");
    constexpr int kM = Q::kKs1 - Sh;   // each member's own k-steps of the first layer
    // at most 4 outputs: the output layer on the VALU leaves output g of pixel j in lane (g, j)
    constexpr bool kVOut = valu_out<S>();
    const int k = bid_y();
    const int lane = tid_x() & 63, wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6), i16 = lane & 15, g = lane >> 4;
    // each wave's LDS exchanges (in place of lane swaps): the tile operands (both members', or the shared k-steps
    // and both members' own), the VALU output layer's reduce-scatters of both members, the pixel sums of both
    // members' errors
    constexpr int kTileLds = Sh > 0 ? 4 * 64 * (Sh + 2 * kM) : 2 * kTilesLds<S>;
    constexpr int kWaveLds = kTileLds + (kVOut ? 2 * kVoTile : 0) + kSumsLds;
    __shared__ __attribute__((aligned(16))) float lds[4 * kWaveLds];
    float* const tl = lds + wave * kWaveLds;
    float* const vo = tl + kTileLds;
    float* const sums = vo + (kVOut ? 2 * kVoTile : 0);
    const __amdgpu_buffer_rsrc_t rz = buffer_of(zdec, 4u * (uint32_t)m.nz), re = buffer_of(eps + (size_t)k * m.nz, 4u * (uint32_t)m.nz),
                                 rn = buffer_of(eps, 0u);   // a level outside the mask: no Gaussians (every load 0)
    float* out = dpix + (size_t)k * m.npix;
    MfmaWeights<S> W;
    mfma_load<S, typename PickType<(Sh > 0), InLatShared<S>, InIdentity>::type>(W, w, lane);
    if constexpr (!Clamp) scale_output<S>(W, kNegLog2e);
    if constexpr (Act == kActFold) scale_hidden<S>(W, fold_scale(m.leak));
    const float ak = act_k_of<Act>(m);
    float cw[4];
    if constexpr (kVOut) {
#pragma unroll
        for (int r = 0; r < 4; r++) cw[r] = (r == 0 && g < NO) ? m.cw[g] : 0.0f;
    } else {
        lane_cw<S>(m.cw, g, cw);
    }
    // the targets of the tile at pixel t0: lane (g, j) reads channels out_at(g, r) of pixel t0 + j (padding
    // reads a valid channel; rows past the last pixel are clamped); VALU output layer: channel g
    auto load_t = [&](int t0, float (&t)[4]) {
        const int pr = min(t0 + i16, m.npix - 1);
        if constexpr (kVOut) {
            t[0] = tgt[(size_t)pr * NO + min(g, NO - 1)];
#pragma unroll
            for (int r = 1; r < 4; r++) t[r] = 0.0f;
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++) t[r] = r < out_regs<S>() ? tgt[(size_t)pr * NO + max(out_at<S>(g, r), 0)] : 0.0f;
        }
    };
    for (int rd = 0; rd < kRounds; rd++) {
        if (rd >= rounds) break;
        const int base = bid_x() * 256 * rounds + 64 * rounds * wave + 64 * rd;   // tile t: pixels base + 16 t + j
        float tn[4];
        load_t(base, tn);
        // both members' first-layer operands (Sh = 0), or the shared k-steps' and each member's own (Sh > 0)
        float bp[4][Sh > 0 ? kM : Q::kKs1], bm[4][Sh > 0 ? kM : Q::kKs1], bs[4][Sh > 0 ? Sh : 1];
        {
            int px, py;
            round_pixel(m, base, lane, px, py);
            if constexpr (Sh > 0) {
                float fs[S::kC0 + 2 * S::kNpos], fp[S::kC1], fm[S::kC1];
                features_lat_shared<S>(m, rz, re, sg, px, py, fs, fp, fm);
                tiles_of_n<Sh>(fs, bs, tl, g, i16);
                tiles_of_n<kM>(fp, bp, tl + 4 * 64 * Sh, g, i16);
                tiles_of_n<kM>(fm, bm, tl + 4 * 64 * (Sh + kM), g, i16);
            } else {
                float fp[S::kMaxIn], fm[S::kMaxIn];
                features_pm<S>(m, rz, re, rn, sg, mask, px, py, fp, fm);
                tiles_of<S>(fp, bp, tl, g, i16);
                tiles_of<S>(fm, bm, tl + kTilesLds<S>, g, i16);
            }
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            float tt[4];
#pragma unroll
            for (int r = 0; r < 4; r++) tt[r] = tn[r];
            if (t + 1 < 4) load_t(base + 16 * (t + 1), tn);
            const int p = base + 16 * t + i16;
            lat_pair_tile<S, Act, Clamp, Sh, UnitCw>(m, W, ak, cw, bs[t], bp[t], bm[t], tt, vo, sums, g, i16, p, out);
        }
    }
}

// The selector search's occupancy target: four waves per SIMD for the 8-input, 32-wide models with more than 4
// outputs and the folded activation, which fit in 128 VGPRs without scratch (the compiler alone gives them 130 and
// three waves); the compiler's choice for the other shapes, several of which spill at four.
template <class S, int Act>
constexpr int qat_occupancy() {
    return (MfmaShape<S>::kIn <= 8 && MfmaShape<S>::kH == 32 && !valu_out<S>() && Act == kActFold) ? 4 : 1;
}

// The selector search (qat_search, main.cpp:2088-2139) on the matrix cores, for a nearest level 0
// of the image's size (each texel's cell is its own pixel): wave = 64 pixels in four 16-pixel tiles.
// Every lane builds the features of its own pixel (features<S>) and tiles_of turns them into the four
// tiles' B operands. Per tile and channel, every candidate value is one MLP evaluation of the tile with
// that feature replaced (two candidates at a time); the first layer's sums over the other inputs are formed
// once per tile and channel and the candidate's term is added to them last (the reference adds it in input
// order, main.cpp:603-627: the same products, one rounding order apart). The choice is the reference's: the current grid
// value first, then every other value with strict <, so the first strictly smaller loss wins
// (main.cpp:2101-2132). The winner enters the features of the next channel and is written to the
// decode buffer. A candidate's loss is the pixel's float sum of cw (d d) over its channels (a lane's
// out_regs, then the pixel's four lanes pairwise, the same value in each of them) with the hidden
// activation of act<Act>: the reference adds the float terms in double with its own activation, so a
// choice can differ from the reference's only between candidates whose losses agree to a few float
// roundings (the reference's own check accepts such rounding ties, main.cpp:3143-3144).
// UnitCw: every channel weight is 1, so a candidate's error terms are d d (fused into the sum where a lane holds several)
template <class S, int Act, bool Clamp, bool UnitCw = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(qat_occupancy<S, Act>()))) k_qat_mfma(DevModel m, const float* __restrict__ w, float* __restrict__ zdec,
                                                 const float* __restrict__ tgt, const int* __restrict__ qat_bits,
                                                 const float* __restrict__ grid) {
    using Q = MfmaShape<S>;
    constexpr int NO = Q::kNout, C0 = S::kC0;
    const int lane = tid_x() & 63, wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6), i16 = lane & 15, g = lane >> 4;
    constexpr bool kVOut = valu_out<S>();   // the output layer on the VALU: output g of pixel j in lane (g, j)
    // each wave's LDS exchanges (in place of lane swaps): the tile operands, the VALU output layer's
    // reduce-scatters of both candidates, the candidates' pixel sums
    constexpr int kWaveLds = kTilesLds<S> + (kVOut ? 2 * kVoTile : 0) + kSumsLds;
    __shared__ __attribute__((aligned(16))) float lds[4 * kWaveLds];
    float* const tl = lds + wave * kWaveLds;
    float* const vo = tl + kTilesLds<S>;
    float* const sums = vo + (kVOut ? 2 * kVoTile : 0);
    MfmaWeights<S> W;
    mfma_load<S>(W, w, lane);
    if constexpr (!Clamp) scale_output<S>(W, kNegLog2e);
    if constexpr (Act == kActFold) scale_hidden<S>(W, fold_scale(m.leak));
    const float ak = act_k_of<Act>(m);
    float cw[4];
    if constexpr (kVOut) {
#pragma unroll
        for (int r = 0; r < 4; r++) cw[r] = (r == 0 && g < NO) ? m.cw[g] : 0.0f;
    } else {
        lane_cw<S>(m.cw, g, cw);
    }
    const int base = bid_x() * 256 + wave * 64;   // tile t: pixels base + 16 t + j
    float f[S::kMaxIn];
    {
        const int pr = min(base + lane, m.npix - 1);
        features<S>(m, PlainLatent{ zdec }, pr % m.W, pr / m.W, f);
    }
    float b[4][Q::kKs1];
    tiles_of<S>(f, b, tl, g, i16);
    // the targets of tile t: lane (g, j) holds channels out_at(g, r) (VALU output layer: g) of pixel j; loaded one
    // tile ahead, so only the first tile's loads are waited for before the search starts
    auto load_t = [&](int t, float (&tv)[4]) {
        const int pr = min(base + 16 * t + i16, m.npix - 1);
#pragma unroll
        for (int r = 0; r < 4; r++) tv[r] = tgt[(size_t)pr * NO + (kVOut ? min(g, NO - 1) : max(out_at<S>(g, r), 0))];
    };
    // per channel: its bit depth, its grid, and the current grid index of the lane's own pixel
    int bits[C0], cur_own[C0];
    const float* gvs[C0];
#pragma unroll
    for (int c = 0; c < C0; c++) {
        bits[c] = qat_bits[c];
        gvs[c] = grid + bits[c] * 257;
        cur_own[c] = qat_index(f[c], bits[c]);
    }
    float tn[4];
    load_t(0, tn);
    // Tile by tile (a tile's pixels are independent of the other tiles'), each tile's channels in order: the winner of
    // channel c enters the features of channel c + 1, as in the reference's per-texel loop.
#pragma unroll
    for (int t = 0; t < 4; t++) {
        float tt[4];
#pragma unroll
        for (int r = 0; r < 4; r++) tt[r] = tn[r];
        if (t + 1 < 4) load_t(t + 1, tn);
#pragma unroll
        for (int c = 0; c < C0; c++) {
            const int levels = (1 << bits[c]) - 1;
            const float* gv = gvs[c];
            // the channel's current index of pixel j of tile t, from the lane that built the pixel's features
            const int cur = __builtin_amdgcn_ds_bpermute((16 * t + i16) << 2, cur_own[c]);
            // the losses and grid values of the current candidate and of the best other one so far: the winner's
            // value comes from these registers, not from a load of the grid after the search
            // best over the other candidates in ascending k, from +inf with a strict <; a NaN loss never wins and a NaN
            // current loss keeps the current value, as the reference's running minimum from the current loss gives
            // (main.cpp:2122-2127). The NaN tests are on the bits: this file is compiled assuming no NaNs.
            // (selects, not branches: the choice is per lane. A best_l still at +inf means no other candidate won.)
            float cur_l = 0.0f, best_l = __builtin_inff(), cur_v = 0.0f, best_v = 0.0f;
            // The first layer's sums of the tile without input c (a zero in its place: fma(w, 0, s) = s) and, in D
            // layout, the weight of input c into each of this lane's units (read from the lane of W.a1 that holds
            // it): a candidate's first-layer pre-activations are then one fused multiply-add, w_c gc + base, and
            // the matrix cores take only the layers after the first for each candidate.
            f4v s1[1][Q::kHt];
            {
                float b0[1][Q::kKs1];
#pragma unroll
                for (int ks = 0; ks < Q::kKs1; ks++) b0[0][ks] = (ks == c / 4 && g == c % 4) ? 0.0f : b[t][ks];
                mfma_layer1<S, 1>(W, b0, s1);
            }
            float w1c[Q::kHt][4];
#pragma unroll
            for (int ot = 0; ot < Q::kHt; ot++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    w1c[ot][r] = __int_as_float(__builtin_amdgcn_ds_bpermute(((c % 4) * 16 + 4 * g + r) << 2, __float_as_int(W.a1[ot][c / 4])));
            for (int kc = 0; kc <= levels; kc += 2) {   // 2^bits candidates: two tiles at a time
                const float gc[2] = { gv[kc], gv[kc + 1] };
                f4v a1[2][Q::kHt];
#pragma unroll
                for (int v = 0; v < 2; v++)
#pragma unroll
                    for (int ot = 0; ot < Q::kHt; ot++)
#pragma unroll
                        for (int r = 0; r < 4; r++) a1[v][ot][r] = __builtin_fmaf(w1c[ot][r], gc[v], s1[0][ot][r]);
                float lv[2];   // this lane's channels, then the pixel's lanes
                float x[2][Q::kKsH];
                mfma_hidden_from1<S, 2, Act>(W, a1, ak, x);
                if constexpr (kVOut) {
#pragma unroll
                    for (int v = 0; v < 2; v++) {
                        const float d = out_of<S>(valu_out_g<S>(W, x[v], vo + v * kVoTile, g, i16), Clamp) - tt[0];
                        constexpr bool kUnit = UnitCw && NO == 4;
                        lv[v] = kUnit ? __fmul_rn(d, d) : __fmul_rn(cw[0], __fmul_rn(d, d));   // cw (d d), main.cpp:2119
                    }
                } else {
                    f4v o[2];
                    mfma_output<S, 2>(W, x, o);
#pragma unroll
                    for (int v = 0; v < 2; v++) {
                        lv[v] = 0.0f;
#pragma unroll
                        for (int r = 0; r < out_regs<S>(); r++) {
                            const float d = out_of<S>(o[v][r], Clamp) - tt[r];
                            constexpr bool kUnit = UnitCw && NO == 4 * out_regs<S>();
                            lv[v] = kUnit ? __builtin_fmaf(d, d, lv[v]) : __builtin_fmaf(cw[r], __fmul_rn(d, d), lv[v]);
                        }
                    }
                }
                float ls[2];
                group_sums(lv[0], lv[1], sums, g, i16, ls[0], ls[1]);
#pragma unroll
                for (int v = 0; v < 2; v++) {
                    const float l = ls[v];
                    const bool is_cur = kc + v == cur;
                    const bool better = !is_cur && not_nan_bits(l) && l < best_l;
                    cur_l = is_cur ? l : cur_l;
                    cur_v = is_cur ? gc[v] : cur_v;
                    best_l = better ? l : best_l;
                    best_v = better ? gc[v] : best_v;
                }
            }
            // cur is in 0 .. levels (qat_index clamps), so cur_v is its grid value
            const float win_v = (not_nan_bits(cur_l) && best_l < cur_l) ? best_v : cur_v;
            if (g == c % 4) b[t][c / 4] = win_v;
            const int p = base + 16 * t + i16;
            if (g == 0 && p < m.npix) zdec[m.lv[0].off + (size_t)p * m.lv[0].C + c] = win_v;
        }
    }
}

}   // namespace ntc_hip
