// Quantizer kernels of the gfx950 ES backend: the --qes snap of the decode copy, and the --dct-q
// level-0 plane (pre-start clamp, snap = forward DCT + quantizer + inverse DCT, reconstruction
// from uploaded symbols, and the --dct-lambda rate proxy of one latent step's pairs).
//
// Strict floating point throughout (this file, like every .hip file, is built with
// -ffp-contract=off, and the quantizers contain no fused operation), so indices, symbols, codes and
// bit counts equal the reference's host functions bit for bit. The one exception is the decoder
// sensitivity probe (an estimate in the reference too), which evaluates the MLP as the decode does. Reference (main.cpp): qes_index /
// qes_snap_level 446-495; dct_clampf .. dct_clamp_level0 783-976; dct_rate_block 884-896.
#include "shapes.hpp"
#include "trainer_impl.hpp"

namespace ntc_hip {

constexpr int kTPB = 256;
constexpr int kTPB_DCT = 64;   // one (block, channel) per thread, 3 x 64 floats of state each

// ---------------------------------------------------------------- --qes
__device__ __forceinline__ int qes_index(float v, float lo, float range, int levels) {
    const float r = rintf(((v - lo) / range) * (float)levels);   // round half to even
    if (!(r == r)) return 0;
    return r <= 0.0f ? 0 : (r >= (float)levels ? levels : (int)r);
}

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
__device__ __forceinline__ int floor_log2(unsigned v) { int k = 0; while (v >>= 1) k++; return k; }
__device__ __forceinline__ int c_run(int r) { return 16 * (2 * floor_log2((unsigned)(r + 1)) + 1); }
__device__ __forceinline__ int c_mag(int q) { return 16 * (2 * floor_log2((unsigned)q) + 1); }
__device__ __forceinline__ int lo_weight(int tok, int p, int lo16) { return p <= 2 ? (tok * lo16 + 8) >> 4 : tok; }

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
// 8x8 transforms with the basis folded in; w[x * 8 + y], C[u * 8 + v]; sums from 0, index ascending
__device__ void fwd8(const DevDct& D, const float* w, float* C) {
    float T[64];
    for (int x = 0; x < 8; x++)
        for (int v = 0; v < 8; v++) { float s = 0.0f; for (int y = 0; y < 8; y++) s = s + w[x * 8 + y] * D.basis[v * 8 + y]; T[x * 8 + v] = s; }
    for (int u = 0; u < 8; u++)
        for (int v = 0; v < 8; v++) { float s = 0.0f; for (int x = 0; x < 8; x++) s = s + T[x * 8 + v] * D.basis[u * 8 + x]; C[u * 8 + v] = s; }
}
__device__ void inv8(const DevDct& D, const float* C, float* w) {
    float T[64];
    for (int x = 0; x < 8; x++)
        for (int v = 0; v < 8; v++) { float s = 0.0f; for (int u = 0; u < 8; u++) s = s + D.basis[u * 8 + x] * C[u * 8 + v]; T[x * 8 + v] = s; }
    for (int x = 0; x < 8; x++)
        for (int y = 0; y < 8; y++) { float s = 0.0f; for (int v = 0; v < 8; v++) s = s + D.basis[v * 8 + y] * T[x * 8 + v]; w[x * 8 + y] = s; }
}
// proxy bits of one (block, channel), 1/16 bit (dct_block_bits)
__device__ int block_bits(const DevDct& D, const int16_t* sym) {
    int bits = 0, run = 0, lnz = 0;
    for (int p = 1; p < 64; p++) {
        const int q = sym[D.zigzag[p]];
        if (q == 0) { run++; continue; }
        bits += lo_weight(c_run(run) + c_mag(min(256, abs(q))) + 16, p, D.lo_w16);
        lnz = p; run = 0;
    }
    if (lnz < 63) bits += 32;
    return bits;
}
// greedy truncation from zigzag 63 down (dct_truncate_block)
__device__ int truncate_block(const DevDct& D, const float* Cf, const int* st, float lam16, int16_t* sym) {
    int ntrunc = 0, next = 64;
    for (int p = 63; p >= 1; p--) {
        const int k = D.zigzag[p], q = sym[k];
        if (q == 0) continue;
        int prev = 0;
        for (int j = p - 1; j >= 1; j--) if (sym[D.zigzag[j]] != 0) { prev = j; break; }
        const int r1 = p - prev - 1;
        const int token = lo_weight(c_run(r1) + c_mag(min(256, abs(q))) + 16, p, D.lo_w16);
        const int saved = next == 64 ? token - (p == 63 ? 32 : 0) : token + c_run(next - p - 1) - c_run(next - p - 1 + r1 + 1);
        const float v = dequant_ac(q, st[k], k / 8, k % 8, D.deadzone != 0), c = Cf[k];
        const float dD = c * c - (c - v) * (c - v);
        if (dD < lam16 * (float)saved) { sym[k] = 0; ntrunc++; }
        else next = p;
    }
    return ntrunc;
}
// dct_quantize_block
__device__ int quantize_block(const DevDct& D, const float* Cf, const int* st, float lam16, bool with_bits, int16_t* sym,
                              int* ntrunc, int* nz_before) {
    for (int k = 0; k < 64; k++) sym[k] = (int16_t)(k == 0 ? quant_dc(Cf[0], D.dc_step) : quant_ac(Cf[k], st[k], k / 8, k % 8, D.deadzone != 0));
    int nt = 0, nz = 0;
    if (lam16 > 0.0f) {
        for (int k = 1; k < 64; k++) if (sym[k] != 0) nz++;
        nt = truncate_block(D, Cf, st, lam16, sym);
    }
    *ntrunc = nt; *nz_before = nz;
    return with_bits ? block_bits(D, sym) : 0;
}
__device__ __forceinline__ size_t lvl0_index(const DevLevel& L0, int bx, int by, int x, int y, int c) {
    return (size_t)L0.off + ((size_t)(by * 8 + y) * L0.W + (bx * 8 + x)) * L0.C + c;
}
// dequantize + inverse DCT + clamp into zq (dct_recon_block)
__device__ void recon_block(const DevDct& D, const DevLevel& L0, int i, const int16_t* sy, const int* st, float* zq) {
    const int b = i / D.C, c = i % D.C, bx = b % D.BW, by = b / D.BW;
    float Cf[64], w[64];
    for (int k = 0; k < 64; k++) Cf[k] = k == 0 ? dequant_dc(sy[0], D.dc_step) : dequant_ac(sy[k], st[k], k / 8, k % 8, D.deadzone != 0);
    inv8(D, Cf, w);
    for (int y = 0; y < 8; y++)
        for (int x = 0; x < 8; x++) zq[lvl0_index(L0, bx, by, x, y, c)] = dct_clampf(w[y * 8 + x] / 32.0f - 1.0f, -1.0f, 1.0f);
}

__global__ void __launch_bounds__(kTPB) k_dct_clamp0(float* __restrict__ z, float* __restrict__ zq, size_t off, size_t n0) {
    const size_t i = (size_t)blockIdx.x * kTPB + threadIdx.x;
    if (i >= n0) return;
    const float v = dct_clampf(z[off + i], -1.0f, 1.0f);
    z[off + i] = v; zq[off + i] = v;
}

// dct_snap_block per (block, channel): clamp the shadow in place, forward DCT of (s + 1) * 32,
// quantize (+ truncation), symbols out, reconstruct zq; integer counters are order-independent.
__global__ void __launch_bounds__(kTPB_DCT) k_dct_snap(DevDct D, DevLevel L0, float* __restrict__ z, float* __restrict__ zq,
                                                      int16_t* __restrict__ sym, const uint8_t* __restrict__ code,
                                                      const int* __restrict__ step, int32_t* __restrict__ bits, int* __restrict__ cnt) {
    const int i = blockIdx.x * kTPB_DCT + threadIdx.x;
    if (i >= D.n) return;
    const int b = i / D.C, c = i % D.C, bx = b % D.BW, by = b / D.BW;
    float w[64], Cf[64];
    for (int y = 0; y < 8; y++)
        for (int x = 0; x < 8; x++) {
            const size_t idx = lvl0_index(L0, bx, by, x, y, c);
            const float s = dct_clampf(z[idx], -1.0f, 1.0f);
            z[idx] = s;
            w[y * 8 + x] = (s + 1.0f) * 32.0f;
        }
    fwd8(D, w, Cf);
    const int cd = code[i];
    const int* st = step + ((size_t)c * 16 + cd) * 64;
    int16_t sy[64];
    int nt = 0, nz = 0;
    quantize_block(D, Cf, st, D.lam_t16[cd], false, sy, &nt, &nz);
    for (int k = 0; k < 64; k++) sym[(size_t)i * 64 + k] = sy[k];
    if (D.rate_es || D.rate_trunc) {
        bits[i] = block_bits(D, sy);
        if (nt) atomicAdd(cnt, nt);
        if (nz) atomicAdd(cnt + 1, nz);
    }
    recon_block(D, L0, i, sy, st, zq);
}

// level 0 of the decode copy from uploaded symbols (the shadow is not touched)
__global__ void __launch_bounds__(kTPB_DCT) k_dct_recon(DevDct D, DevLevel L0, const int16_t* __restrict__ sym,
                                                       const uint8_t* __restrict__ code, const int* __restrict__ step,
                                                       float* __restrict__ zq, int32_t* __restrict__ bits) {
    const int i = blockIdx.x * kTPB_DCT + threadIdx.x;
    if (i >= D.n) return;
    int16_t sy[64];
    for (int k = 0; k < 64; k++) sy[k] = sym[(size_t)i * 64 + k];
    if (D.rate_es || D.rate_trunc) bits[i] = block_bits(D, sy);
    recon_block(D, L0, i, sy, step + ((size_t)(i % D.C) * 16 + code[i]) * 64, zq);
}

// --dct-lambda part A for pair blockIdx.y: bits(snap(clamp(z + sg eps))) - bits(snap(clamp(z - sg eps)))
// on the shadow, with the pair's level-0 Gaussians (the latent step's own draws).
__global__ void __launch_bounds__(kTPB_DCT) k_dct_rate_pair(DevDct D, DevLevel L0, long long nz, float sg,
                                                           const float* __restrict__ z, const float* __restrict__ eps,
                                                           const uint8_t* __restrict__ code, const int* __restrict__ step,
                                                           int32_t* __restrict__ dbits, int* __restrict__ hits) {
    const int i = blockIdx.x * kTPB_DCT + threadIdx.x;
    if (i >= D.n) return;
    const int k = blockIdx.y;
    const float* e = eps + (size_t)k * nz;
    const int b = i / D.C, c = i % D.C, bx = b % D.BW, by = b / D.BW;
    const int cd = code[i];
    const int* st = step + ((size_t)c * 16 + cd) * 64;
    const float lam = D.lam_t16[cd];
    int bb[2];
    for (int sgn = 0; sgn < 2; sgn++) {
        float w[64], Cf[64];
        int16_t sy[64];
        for (int y = 0; y < 8; y++)
            for (int x = 0; x < 8; x++) {
                const size_t idx = lvl0_index(L0, bx, by, x, y, c);
                const float pert = sg * e[idx];
                const float s = dct_clampf(sgn == 0 ? z[idx] + pert : z[idx] - pert, -1.0f, 1.0f);
                w[y * 8 + x] = (s + 1.0f) * 32.0f;
            }
        fwd8(D, w, Cf);
        int nt, nzb;
        bb[sgn] = quantize_block(D, Cf, st, lam, true, sy, &nt, &nzb);
    }
    dbits[(size_t)k * D.n + i] = bb[0] - bb[1];
    if (bb[0] != bb[1]) atomicAdd(hits, 1);
}

// z += f * (zq - z) on [off, off + n) (one fused operation, as the reference's build evaluates
// main.cpp:4144)
__global__ void __launch_bounds__(kTPB) k_shadow_pull(float* __restrict__ z, const float* __restrict__ zq, size_t off, size_t n, float f) {
    const size_t i = (size_t)blockIdx.x * kTPB + threadIdx.x;
    if (i < n) z[off + i] = __builtin_fmaf(f, zq[off + i] - z[off + i], z[off + i]);
}

__global__ void k_zero_ints(int* __restrict__ p, int n) {
    const int i = threadIdx.x;
    if (i < n) p[i] = 0;
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
// The decoder sensitivity probe of a DCT-coded level 0 (dct_probe_codes, main.cpp:1001-1032), on the
// device: one thread per (block, channel). At the 4 positions (8 bx + {2, 5}, 8 by + {2, 5}) the
// features are built once from the decode buffer and the MLP evaluated with level-0 channel c set to
// -1, -0.5, 0, 0.5, 1; segment gain g = (255 / 16) sqrt(sum_o cw_o (out_{j+1} - out_j)^2 / wsum), block
// gain = RMS over the 16 (position, segment) pairs, code = round(log2(g / g_floor) / 0.6) in [0, 15].
// The reference calls the probe an estimate (not strict FP): the device's expf and log2 can move a
// gain that sits on a code boundary to the neighbouring code.
template <class S>
__global__ void __launch_bounds__(kTPB_DCT) k_dct_probe(DevModel m, const float* __restrict__ w, const float* __restrict__ zdec,
                                                       int BW, int BH, int C, uint8_t* __restrict__ code, float* __restrict__ gain) {
    const int t = blockIdx.x * kTPB_DCT + threadIdx.x;
    if (t >= BW * BH * C) return;
    const int c = t % C, b = t / C, bx = b % BW, by = b / BW;
    const int P[2] = { 2, 5 };
    const float SJ[5] = { -1.0f, -0.5f, 0.0f, 0.5f, 1.0f };
    double acc = 0.0;
    for (int py = 0; py < 2; py++)
        for (int px = 0; px < 2; px++) {
            float f[S::kMaxIn], out[5][S::kMaxOut];
            features<S>(m, PlainLatent{ zdec }, bx * 8 + P[px], by * 8 + P[py], f);
            for (int j = 0; j < 5; j++) {
                f[c] = SJ[j];
                mlp_forward<S>(m, w, f, out[j]);
            }
            for (int j = 0; j < 4; j++) {
                double ss = 0.0;
                for (int o = 0; o < m.nout; o++) {
                    const double d = (double)out[j + 1][o] - (double)out[j][o];
                    ss = __dadd_rn(ss, __dmul_rn(__dmul_rn((double)m.cw[o], d), d));
                }
                const double g = (255.0 / 16.0) * sqrt(ss / (double)m.wsum);
                acc += g * g;
            }
        }
    const double gb = sqrt(acc / 16.0);
    const double gf = 14.0 / 64.0;
    const double gc = gb > gf ? gb : gf;
    const long long k = (long long)round(log2(gc / gf) / 0.6);
    code[t] = (uint8_t)(k < 0 ? 0 : (k > 15 ? 15 : k));
    if (gain) gain[t] = (float)gb;
}

void launch_dct_snap(Impl& I) {
    ProfScope ps(I, "dct_snap");
    if (I.dct_rate_es || I.dct_rate_trunc) {
        hipLaunchKernelGGL(k_zero_ints, dim3(1), dim3(64), 0, I.stream, I.dct_cnt, 2);
        NTC_CHECK(hipGetLastError());
    }
    hipLaunchKernelGGL(k_dct_snap, dim3(blocks_for(I.ddct.n, kTPB_DCT)), dim3(kTPB_DCT), 0, I.stream, I.ddct, I.dm.lv[0], I.z, I.zq,
                       I.dct_sym, I.dct_code, I.dct_step, I.dct_bits, I.dct_cnt);
    NTC_CHECK(hipGetLastError());
}
void launch_dct_recon(Impl& I) {
    hipLaunchKernelGGL(k_dct_recon, dim3(blocks_for(I.ddct.n, kTPB_DCT)), dim3(kTPB_DCT), 0, I.stream, I.ddct, I.dm.lv[0], I.dct_sym,
                       I.dct_code, I.dct_step, I.zq, I.dct_bits);
    NTC_CHECK(hipGetLastError());
}
void launch_dct_rate_pairs(Impl& I, int K, float sigma) {
    ProfScope ps(I, "dct_rate");
    hipLaunchKernelGGL(k_zero_ints, dim3(1), dim3(64), 0, I.stream, I.dct_cnt + 2, 1);
    NTC_CHECK(hipGetLastError());
    hipLaunchKernelGGL(k_dct_rate_pair, dim3(blocks_for(I.ddct.n, kTPB_DCT), K), dim3(kTPB_DCT), 0, I.stream, I.ddct, I.dm.lv[0],
                       (long long)I.nz, sigma, I.z, I.eps_lat, I.dct_code, I.dct_step, I.dct_dbits, I.dct_cnt + 2);
    NTC_CHECK(hipGetLastError());
}
void launch_shadow_pull(Impl& I, size_t off, size_t n, float f) {
    hipLaunchKernelGGL(k_shadow_pull, dim3(blocks_for(n, kTPB)), dim3(kTPB), 0, I.stream, I.z, I.zq, off, n, f);
    NTC_CHECK(hipGetLastError());
}

void launch_dct_probe(Impl& I, uint8_t* code, float* gain) {
    ProfScope ps(I, "dct_probe");
    dispatch_shape(I.dm, [&](auto s) {
        using S = decltype(s);
        hipLaunchKernelGGL(k_dct_probe<S>, dim3(blocks_for(I.ddct.n, kTPB_DCT)), dim3(kTPB_DCT), 0, I.stream, I.dm, I.w, I.zdec,
                           I.ddct.BW, I.ddct.BH, I.ddct.C, code, gain);
    });
    NTC_CHECK(hipGetLastError());
}

}   // namespace ntc_hip
