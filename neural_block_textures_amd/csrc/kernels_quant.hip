// Quantizer kernels of the gfx950 ES backend: the --qes snap of the decode copy, and the --dct-q
// level-0 plane (pre-start clamp, snap = forward DCT + quantizer + inverse DCT, reconstruction
// from uploaded symbols, and the --dct-lambda rate proxy of one latent step's pairs).
//
// Strict floating point throughout (this file, like every .hip file, is built with
// -ffp-contract=off, and the quantizers contain no fused operation), so indices, symbols, codes and
// bit counts equal the reference's host functions bit for bit. The one exception is the decoder
// sensitivity probe (an estimate in the reference too), which evaluates the MLP as the decode does. Reference (main.cpp): qes_index /
// qes_snap_level 446-495; dct_clampf .. dct_clamp_level0 783-976; dct_rate_block 884-896.
#include "kern_valu.hpp"
#include "jit.hpp"
#include "shapes.hpp"
#include "trainer_impl.hpp"

namespace ntc_hip {


// ---------------------------------------------------------------- --qes (qes_index: device_common.hpp)

// zq = snap(z) per level (a level without --qes bits is copied); once frozen the shadow is first
// clamped to [lo, hi] (std::min(std::max(v, lo), hi) semantics) and written back.
__global__ void __launch_bounds__(kTPB) k_qes_snap(DevModel m, const ntc_cuda::QesDesc* __restrict__ q,
                                                  const float* __restrict__ grid, float* __restrict__ z, float* __restrict__ zq) {
    const long long i = (long long)blockIdx.x * kTPB + threadIdx.x;
    if (i >= m.nz) return;
    int l = 0;
    for (int r = 1; r < m.nlev; r++) if (i >= m.lv[r].off) l = r;
    const int bits = q->live ? q->bits[l] : 0;
    float v = z[i];
    if (bits == 0) { zq[i] = v; return; }
    const int c = (int)((i - m.lv[l].off) % m.lv[l].C);
    const float lo = q->lo[l][c], hi = q->hi[l][c];
    if (q->frozen) { v = (v < lo) ? lo : v; v = (hi < v) ? hi : v; z[i] = v; }
    const int levels = (1 << bits) - 1;
    zq[i] = grid[q->grid_off[l][c] + qes_index(v, lo, q->range[l][c], levels)];
}

// ---------------------------------------------------------------- --dct-q
__device__ __forceinline__ float dct_clampf(float v, float lo, float hi) { if (!(v >= lo)) return lo; if (v > hi) return hi; return v; }
__device__ __forceinline__ bool first_order(int u, int v) { return (u == 1 && v == 0) || (u == 0 && v == 1); }

__device__ __forceinline__ int quant_dc(float d, int S) { return (int)dct_clampf(rintf(d / (float)S), -1024.0f, 1024.0f); }
__device__ __forceinline__ float dequant_dc(int q, int S) { return (float)q * (float)S; }
__device__ __forceinline__ int quant_ac(float d, int L, int u, int v, bool dz) {
    if (!dz || first_order(u, v)) return (int)dct_clampf(roundf(d / (float)L), -1024.0f, 1024.0f);
    const float s = fabsf(d), tau = 0.5f * (float)L;
    if (s <= tau) return 0;
    const float qf = (s - tau) / (float)L;
    const int q = (int)dct_clampf(floorf(qf + 0.5f), 0.0f, 1024.0f);
    return d < 0.0f ? -q : q;
}
__device__ __forceinline__ float dequant_ac(int q, int L, int u, int v, bool dz) {
    if (!dz || first_order(u, v)) return (float)q * (float)L;
    if (q == 0) return 0.0f;
    const float tau = 0.5f * (float)L;
    const float mag = tau + (float)abs(q) * (float)L;
    return q < 0 ? -mag : mag;
}
__device__ __forceinline__ size_t lvl0_index(const DevLevel& L0, int bx, int by, int x, int y, int c) {
    return (size_t)L0.off + ((size_t)(by * 8 + y) * L0.W + (bx * 8 + x)) * L0.C + c;
}

// ---- one wave per (block, channel): lane = 8 row + column of the block, or 8 u + v of its
// coefficients, or a zigzag position. Every value is computed with the reference's operations in
// the reference's order (dct_fwd8 / dct_inv8 sums from 0 in ascending index, the quantizers, the
// greedy truncation walking the nonzero ACs from zigzag 63 down, the token costs); only the work is
// spread over the lanes, and the integer totals are order-free.
constexpr int kDctWaves = 4;   // (block, channel) items per 256-thread workgroup

struct DctTables {
    float basis[64];   // [u * 8 + x]
    int zz[64];        // zigzag position -> natural index
    int izz[64];       // natural index -> zigzag position
};
__device__ __forceinline__ void load_tables(const DevDct& D, DctTables& T) {
    if (threadIdx.x < 64) {
        const int t = threadIdx.x;
        T.basis[t] = D.basis[t];
        T.zz[t] = D.zigzag[t];
        T.izz[D.zigzag[t]] = t;
    }
    __syncthreads();
}
__device__ __forceinline__ float lane_f(float v, int src) { return __shfl(v, src); }
__device__ __forceinline__ int readlane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ int ilog2(unsigned v) { return 31 - __clz((int)v); }   // v >= 1
__device__ __forceinline__ int c_run(int r) { return 16 * (2 * ilog2((unsigned)(r + 1)) + 1); }
__device__ __forceinline__ int c_mag(int q) { return 16 * (2 * ilog2((unsigned)q) + 1); }
__device__ __forceinline__ int lo_weight(int tok, int p, int lo16) { return p <= 2 ? (tok * lo16 + 8) >> 4 : tok; }
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// dct_fwd8 (main.cpp:783-789): in lane 8 a + b the sample W[a][b]; out in lane 8 u + v the coefficient
// C[u][v]. T[a][v] = sum_b W[a][b] B[v][b], then C[u][v] = sum_a T[a][v] B[u][a].
__device__ __forceinline__ float wave_fwd8(const DctTables& T, float w, int lane) {
    const int hi = lane >> 3, lo = lane & 7;
    float t = 0.0f;
#pragma unroll
    for (int b = 0; b < 8; b++) t = t + lane_f(w, 8 * hi + b) * T.basis[lo * 8 + b];
    float c = 0.0f;
#pragma unroll
    for (int a = 0; a < 8; a++) c = c + lane_f(t, 8 * a + lo) * T.basis[hi * 8 + a];
    return c;
}
// dct_inv8 (main.cpp:790-796): in lane 8 u + v the coefficient; out in lane 8 a + b the sample. T[a][v] = sum_u B[u][a] C[u][v],
// then W[a][b] = sum_v B[v][b] T[a][v].
__device__ __forceinline__ float wave_inv8(const DctTables& T, float c, int lane) {
    const int hi = lane >> 3, lo = lane & 7;
    float t = 0.0f;
#pragma unroll
    for (int u = 0; u < 8; u++) t = t + T.basis[u * 8 + hi] * lane_f(c, 8 * u + lo);
    float w = 0.0f;
#pragma unroll
    for (int v = 0; v < 8; v++) w = w + T.basis[v * 8 + lo] * lane_f(t, 8 * hi + v);
    return w;
}

// dct_block_bits (main.cpp:835-849) of the symbols whose nonzero ACs are the set bits of m (zigzag
// positions), lane p holding the symbol at position p: each nonzero's token cost with its run since the
// previous nonzero, plus the EOB unless position 63 is the last nonzero.
__device__ __forceinline__ int wave_block_bits(uint64_t m, int qp, int lo16, int lane) {
    int cost = 0;
    if ((m >> lane) & 1ull) {
        const uint64_t below = m & ((1ull << lane) - 1ull);
        const int prev = below ? 63 - __clzll((long long)below) : 0;
        cost = lo_weight(c_run(lane - prev - 1) + c_mag(min(256, abs(qp))) + 16, lane, lo16);
    }
    const int lnz = m ? 63 - __clzll((long long)m) : 0;
    return wave_sum_i(cost) + (lnz < 63 ? 32 : 0);
}

struct WaveSyms { int q; int bits; int ntrunc; int nz; };   // q: this lane's symbol, natural order (lane = k)

// dct_quantize_block (main.cpp:871-883): the symbols of coefficient C (lane = k), the greedy truncation
// with lam16 > 0 (dct_truncate_block, main.cpp:850-870), and the proxy bits of the result when asked.
__device__ WaveSyms wave_quantize(const DevDct& D, const DctTables& T, float Cf, const int* __restrict__ st, float lam16,
                                  bool with_bits, int lane) {
    const bool dz = D.deadzone != 0;
    WaveSyms r;
    r.q = lane == 0 ? quant_dc(Cf, D.dc_step) : quant_ac(Cf, st[lane], lane >> 3, lane & 7, dz);
    // the zigzag view: lane p holds position p
    const int kp = T.zz[lane];
    const int qp = __shfl(r.q, kp);
    uint64_t m = __ballot(lane >= 1 && qp != 0);
    r.nz = lam16 > 0.0f ? __popcll(m) : 0;   // the nonzero ACs before truncation, counted where it runs
    r.ntrunc = 0;
    if (lam16 > 0.0f && m) {
        const float cp = lane_f(Cf, kp);
        const uint64_t below = m & ((1ull << lane) - 1ull);
        const int prev = below ? 63 - __clzll((long long)below) : 0;
        const int r1 = lane - prev - 1;
        const int token = lo_weight(c_run(r1) + c_mag(min(256, abs(qp))) + 16, lane, D.lo_w16);
        const float vq = dequant_ac(qp, st[kp], kp >> 3, kp & 7, dz);
        const float dD = cp * cp - (cp - vq) * (cp - vq);
        uint64_t mm = m, cut = 0;
        int next = 64;
        // Every nonzero's decision at once, as if every nonzero above it were kept: its next kept nonzero is
        // then the nearest nonzero above it. Walking down from the top, that holds until the first cut, so
        // the highest speculative cut is the walk's first cut and every decision above it is the walk's.
        // Cuts are rare (most blocks have none): the walk below resumes only after a cut.
        {
            const uint64_t above = m & ~((2ull << lane) - 1ull);   // lane 63: 2 << 63 wraps to 0, nothing above
            const int nx = above ? __builtin_ctzll(above) : 64;
            const int sv = nx == 64 ? token - (lane == 63 ? 32 : 0) : token + c_run(nx - lane - 1) - c_run(nx - lane - 1 + r1 + 1);
            const uint64_t cm = __ballot(((m >> lane) & 1ull) && dD < lam16 * (float)sv);
            if (cm) {
                const int p = 63 - __clzll((long long)cm);
                cut = 1ull << p;
                r.ntrunc = 1;
                next = readlane_i(nx, p);   // p is cut: the next kept nonzero above the positions below it
                mm = m & ((1ull << p) - 1ull);
            } else {
                mm = 0;
            }
        }
        while (mm) {   // uniform: the wave walks the remaining nonzero ACs from the top
            const int p = 63 - __clzll((long long)mm);
            mm &= ~(1ull << p);
            const int tok = readlane_i(token, p), rr = readlane_i(r1, p);
            const float dd = __int_as_float(readlane_i(__float_as_int(dD), p));
            const int saved = next == 64 ? tok - (p == 63 ? 32 : 0) : tok + c_run(next - p - 1) - c_run(next - p - 1 + rr + 1);
            if (dd < lam16 * (float)saved) { cut |= 1ull << p; r.ntrunc++; }
            else next = p;
        }
        if ((cut >> T.izz[lane]) & 1ull) r.q = 0;
        m &= ~cut;
    }
    r.bits = with_bits ? wave_block_bits(m, qp, D.lo_w16, lane) : 0;
    return r;
}

// dct_recon_block (main.cpp:899-917) of one lane's symbol (natural order): dequantize, inverse DCT, and
// the plane value of this lane's texel (row lane >> 3, column lane & 7)
__device__ __forceinline__ float wave_recon(const DevDct& D, const DctTables& T, int q, const int* __restrict__ st, int lane) {
    const float Cd = lane == 0 ? dequant_dc(q, D.dc_step) : dequant_ac(q, st[lane], lane >> 3, lane & 7, D.deadzone != 0);
    const float w = wave_inv8(T, Cd, lane);
    return dct_clampf(w / 32.0f - 1.0f, -1.0f, 1.0f);
}

__global__ void __launch_bounds__(kTPB) k_dct_clamp0(float* __restrict__ z, float* __restrict__ zq, size_t off, size_t n0) {
    const size_t i = (size_t)blockIdx.x * kTPB + threadIdx.x;
    if (i >= n0) return;
    const float v = dct_clampf(z[off + i], -1.0f, 1.0f);
    z[off + i] = v; zq[off + i] = v;
}

// dct_snap_block (main.cpp:918-940) per (block, channel), one wave each: clamp the shadow in place, forward DCT of
// (s + 1) * 32, quantize (+ truncation), symbols out, reconstruct zq; with the rate term on, the block's
// proxy bits and its two counts (added up on the host when asked: no atomics). pull != 0: the shadow is first pulled
// toward the current plane, z + pull (zq - z) as k_shadow_pull computes it (--dct-shadow-pull followed by the re-snap,
// main.cpp:4142-4146, in one launch: each value of the plane belongs to one wave, which reads its zq before
// replacing it).
__global__ void __launch_bounds__(64 * kDctWaves) k_dct_snap(DevDct D, DevLevel L0, float* __restrict__ z, float* __restrict__ zq,
                                                            int16_t* __restrict__ sym, const uint8_t* __restrict__ code,
                                                            const int* __restrict__ step, int32_t* __restrict__ bits,
                                                            int* __restrict__ tn, float pull) {
    __shared__ DctTables T;
    load_tables(D, T);
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * kDctWaves + (threadIdx.x >> 6);
    if (i >= D.n) return;
    const int b = i / D.C, c = i % D.C, bx = b % D.BW, by = b / D.BW;
    const size_t idx = lvl0_index(L0, bx, by, lane & 7, lane >> 3, c);
    float zv = z[idx];
    if (pull != 0.0f) zv = __builtin_fmaf(pull, zq[idx] - zv, zv);
    const float s = dct_clampf(zv, -1.0f, 1.0f);
    z[idx] = s;
    const float Cf = wave_fwd8(T, (s + 1.0f) * 32.0f, lane);
    const int cd = code[i];
    const int* st = step + ((size_t)c * 16 + cd) * 64;
    const bool rate = D.rate_es || D.rate_trunc;
    const WaveSyms q = wave_quantize(D, T, Cf, st, D.lam_t16[cd], rate, lane);
    sym[(size_t)i * 64 + lane] = (int16_t)q.q;
    if (rate && lane == 0) {
        bits[i] = q.bits;
        tn[i] = q.ntrunc;
        tn[D.n + i] = q.nz;
    }
    zq[idx] = wave_recon(D, T, q.q, st, lane);
}

// level 0 of the decode copy from uploaded symbols (the shadow is not touched)
__global__ void __launch_bounds__(64 * kDctWaves) k_dct_recon(DevDct D, DevLevel L0, const int16_t* __restrict__ sym,
                                                             const uint8_t* __restrict__ code, const int* __restrict__ step,
                                                             float* __restrict__ zq, int32_t* __restrict__ bits) {
    __shared__ DctTables T;
    load_tables(D, T);
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * kDctWaves + (threadIdx.x >> 6);
    if (i >= D.n) return;
    const int q = sym[(size_t)i * 64 + lane];
    if (D.rate_es || D.rate_trunc) {
        const int qp = __shfl(q, T.zz[lane]);
        const int bb = wave_block_bits(__ballot(lane >= 1 && qp != 0), qp, D.lo_w16, lane);
        if (lane == 0) bits[i] = bb;
    }
    const int b = i / D.C, c = i % D.C, bx = b % D.BW, by = b / D.BW;
    zq[lvl0_index(L0, bx, by, lane & 7, lane >> 3, c)] = wave_recon(D, T, q, step + ((size_t)c * 16 + code[i]) * 64, lane);
}

// --dct-lambda part A for pair blockIdx.y: bits(snap(clamp(z + sg eps))) - bits(snap(clamp(z - sg eps)))
// on the shadow, with the pair's level-0 Gaussians (the latent step's own draws); one wave per
// (block, channel, pair). The hit count (pairs whose bits differ) is the number of nonzero dbits.
__global__ void __launch_bounds__(64 * kDctWaves) k_dct_rate_pair(DevDct D, DevLevel L0, long long nz, float sg,
                                                                 const float* __restrict__ z, const float* __restrict__ eps,
                                                                 const uint8_t* __restrict__ code, const int* __restrict__ step,
                                                                 int32_t* __restrict__ dbits) {
    __shared__ DctTables T;
    load_tables(D, T);
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * kDctWaves + (threadIdx.x >> 6);
    if (i >= D.n) return;
    const int k = blockIdx.y;
    const float* e = eps + (size_t)k * nz;
    const int b = i / D.C, c = i % D.C, bx = b % D.BW, by = b / D.BW;
    const int cd = code[i];
    const int* st = step + ((size_t)c * 16 + cd) * 64;
    const float lam = D.lam_t16[cd];
    const size_t idx = lvl0_index(L0, bx, by, lane & 7, lane >> 3, c);
    const float zv = z[idx], pert = sg * e[idx];
    int bb[2];
#pragma unroll
    for (int sgn = 0; sgn < 2; sgn++) {
        const float s = dct_clampf(sgn == 0 ? zv + pert : zv - pert, -1.0f, 1.0f);
        const float Cf = wave_fwd8(T, (s + 1.0f) * 32.0f, lane);
        bb[sgn] = wave_quantize(D, T, Cf, st, lam, true, lane).bits;
    }
    if (lane == 0) dbits[(size_t)k * D.n + i] = bb[0] - bb[1];
}

// z += f * (zq - z) on [off, off + n) (one fused operation, as the reference's build evaluates
// main.cpp:4144)
__global__ void __launch_bounds__(kTPB) k_shadow_pull(float* __restrict__ z, const float* __restrict__ zq, size_t off, size_t n, float f) {
    const size_t i = (size_t)blockIdx.x * kTPB + threadIdx.x;
    if (i < n) z[off + i] = __builtin_fmaf(f, zq[off + i] - z[off + i], z[off + i]);
}

// ---------------------------------------------------------------- launchers
void launch_qes_snap(Impl& I) {
    ProfScope ps(I, "qes_snap");
    hipLaunchKernelGGL(k_qes_snap, dim3(blocks_for(I.nz, kTPB)), dim3(kTPB), 0, I.stream, I.dm, I.qes_dev, I.qgrid, I.z, I.zq);
    NTC_CHECK(hipGetLastError());
}
void launch_dct_clamp0(Impl& I) {
    const size_t n0 = (size_t)I.d.lv[0].W * I.d.lv[0].H * I.d.lv[0].C;
    hipLaunchKernelGGL(k_dct_clamp0, dim3(blocks_for(n0, kTPB)), dim3(kTPB), 0, I.stream, I.z, I.zq, (size_t)I.d.lv[0].off, n0);
    NTC_CHECK(hipGetLastError());
}
void launch_dct_snap(Impl& I, float pull) {
    ProfScope ps(I, "dct_snap");
    hipLaunchKernelGGL(k_dct_snap, dim3(blocks_for(I.ddct.n, kDctWaves)), dim3(64 * kDctWaves), 0, I.stream, I.ddct, I.dm.lv[0], I.z, I.zq,
                       I.dct_sym, I.dct_code, I.dct_step, I.dct_bits, I.dct_tn, pull);
    NTC_CHECK(hipGetLastError());
}
void launch_dct_recon(Impl& I) {
    hipLaunchKernelGGL(k_dct_recon, dim3(blocks_for(I.ddct.n, kDctWaves)), dim3(64 * kDctWaves), 0, I.stream, I.ddct, I.dm.lv[0], I.dct_sym,
                       I.dct_code, I.dct_step, I.zq, I.dct_bits);
    NTC_CHECK(hipGetLastError());
}
void launch_dct_rate_pairs(Impl& I, int k0, int K, float sigma) {
    ProfScope ps(I, "dct_rate");
    hipLaunchKernelGGL(k_dct_rate_pair, dim3(blocks_for(I.ddct.n, kDctWaves), K), dim3(64 * kDctWaves), 0, I.stream, I.ddct, I.dm.lv[0],
                       (long long)I.nz, sigma, I.z, I.eps_lat, I.dct_code, I.dct_step, I.dct_dbits + (size_t)k0 * I.ddct.n);
    NTC_CHECK(hipGetLastError());
}
void launch_shadow_pull(Impl& I, size_t off, size_t n, float f) {
    ProfScope ps(I, "shadow_pull");
    hipLaunchKernelGGL(k_shadow_pull, dim3(blocks_for(n, kTPB)), dim3(kTPB), 0, I.stream, I.z, I.zq, off, n, f);
    NTC_CHECK(hipGetLastError());
}

void launch_dct_probe(Impl& I, uint8_t* code, float* gain) {
    ProfScope ps(I, "dct_probe");
    if (I.jit) {
        jit_launch(k_dct_probe<ShapeDefault>, I, "k_dct_probe", "", dim3(blocks_for(I.ddct.n, kTPB_DCT)), dim3(kTPB_DCT), 0, I.dm, I.w,
                   I.zdec, I.ddct.BW, I.ddct.BH, I.ddct.C, code, gain);
    } else dispatch_shape(I.dm, [&](auto s) {
        using S = decltype(s);
        hipLaunchKernelGGL(k_dct_probe<S>, dim3(blocks_for(I.ddct.n, kTPB_DCT)), dim3(kTPB_DCT), 0, I.stream, I.dm, I.w, I.zdec,
                           I.ddct.BW, I.ddct.BH, I.ddct.C, code, gain);
    });
    NTC_CHECK(hipGetLastError());
}

}   // namespace ntc_hip
