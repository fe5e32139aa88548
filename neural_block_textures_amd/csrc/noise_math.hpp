// The two factors of the Box-Muller draw (cuda/ntc_noise.h:42-47), evaluated in double precision
// with the same operations on the host and on the device.
//
// The reference draws sqrtf(-2 logf(u1)) * cosf(2 pi u2) with the host C library, u1 = (k1 + 1) / 2^24,
// u2 = k2 / 2^24. Over the 2^24 values of each argument, logf and cosf of glibc differ from the
// correctly rounded result on 122,123 and 217,508 inputs, always by one float, on the side of the
// exact value. Here each factor is computed in double from a small table (accurate to a few units in the
// last place of a double: rounded to float it is the correctly rounded value on every argument), and
// moved to the float neighbour on the side of the double value wherever a per-argument bit (built once on
// the host from its own C library, 2 MiB per factor) says the host differs. The host verifies at set-up
// that this rule reproduces its C library on every argument; the result is the host's draw bit for bit.
//
// Only IEEE operations that round identically on x86-64 and gfx950 are used: +, -, *, fma and
// round-to-nearest-even, no library functions; the tables they read are built on the host and copied to the device.
#pragma once
#ifdef __HIPCC_RTC__   // hipRTC provides the runtime itself and the fixed-width integer types in its own namespace
using __hip_internal::int8_t; using __hip_internal::int16_t; using __hip_internal::int32_t; using __hip_internal::int64_t;
using __hip_internal::uint8_t; using __hip_internal::uint16_t; using __hip_internal::uint32_t; using __hip_internal::uint64_t;
#else
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

namespace ntc_hip {

// The tables of the two factors (built once on the host by nm_fill_tables, identical on host and device):
// log: for bin i of the mantissa 1.f of k + 1 (i = the top 7 bits of f), the reciprocal rc of a point c of the bin,
// rounded to double, and -ln(rc); bins from kNmLogSplit on stand for m / 2 (the point and reciprocal halved and doubled),
// bin 0 and the last bin have c = 1 exactly. cos: cos and sin of j 2 pi / 256 for j = 0 .. 256, the quarter points
// exactly 0 and +-1.
constexpr int kNmLogBins = 128, kNmLogSplit = 53, kNmCosSteps = 256;
constexpr int kNmLogTab = 2 * kNmLogBins, kNmCosTab = 2 * (kNmCosSteps + 1);

// ln((k + 1) / 2^24) for k < 2^24: n = k + 1 = 2^e m with m in [1, 2), taken as m / 2 from 1 + 53/128 on (so that m
// near 1 from either side carries no ln 2 term); ln m = -ln rc + ln(1 + r), r = m rc - 1 (one rounding, |r| <= 2^-7),
// ln(1 + r) as its series to r^7.
__host__ __device__ inline double nm_log_u1(uint32_t k, const double* __restrict__ tab) {
    const uint32_t n = k + 1;
    const int e = 31 - __builtin_clz(n);
    const int i = (int)(((n << (31 - e)) >> 24) & 127u);
    const int ee = e + (i >= kNmLogSplit ? 1 : 0);
    const double m = (double)n * __builtin_bit_cast(double, (uint64_t)(1023 - ee) << 52);   // n 2^-ee, exact
    const double r = __builtin_fma(m, tab[2 * i], -1.0);
    double q = 1.0 / 7.0;
    q = __builtin_fma(q, r, -1.0 / 6.0); q = __builtin_fma(q, r, 1.0 / 5.0); q = __builtin_fma(q, r, -1.0 / 4.0);
    q = __builtin_fma(q, r, 1.0 / 3.0); q = __builtin_fma(q, r, -0.5);
    const double lm = __builtin_fma(r * r, q, r);
    const double E = (double)(ee - 24);
    // ln 2 split so that E ln2_hi is exact
    return __builtin_fma(E, 6.93147180369123816490e-01, __builtin_fma(E, 1.90821492927058770002e-10, tab[2 * i + 1] + lm));
}

// cos(x) for a float x in [0, 2 pi): x = j 2 pi / 256 + b with 2 pi / 256 in three parts (the first two with 33
// significant bits, so j times them is exact), |b| <= pi / 256, then cos(j 2 pi / 256) cos b - sin(j 2 pi / 256) sin b
// with cos b to b^6 and sin b to b^5.
__host__ __device__ inline double nm_cos(float x, const double* __restrict__ tab) {
    const double xd = x;
    const double nd = __builtin_rint(xd * 40.74366543152520595683);   // 256 / (2 pi)
    const int j = (int)nd;
    double b = __builtin_fma(-nd, 1.57079632673412561417e+00 / 64.0, xd);
    b = __builtin_fma(-nd, 6.07710050630396597660e-11 / 64.0, b);
    b = __builtin_fma(-nd, 2.02226624879595063154e-21 / 64.0, b);
    const double b2 = b * b;
    const double cb = __builtin_fma(b2, __builtin_fma(b2, __builtin_fma(b2, -1.0 / 720.0, 1.0 / 24.0), -0.5), 1.0);
    const double sb = __builtin_fma(b * b2, __builtin_fma(b2, 1.0 / 120.0, -1.0 / 6.0), b);
    return __builtin_fma(tab[2 * j], cb, -(tab[2 * j + 1] * sb));
}

// the float next to f on the side of d (f nonzero)
__host__ __device__ inline float nm_toward(float f, double d) {
    uint32_t b = __builtin_bit_cast(uint32_t, f);
    const bool up = d > (double)f;
    b = ((f > 0.0f) == up) ? b + 1 : b - 1;
    return __builtin_bit_cast(float, b);
}

// the arguments of the two factors, as the reference forms them
__host__ __device__ inline float nm_u1(uint32_t k1) { return (float)(k1 + 1) * (1.0f / 16777216.0f); }
__host__ __device__ inline float nm_angle(uint32_t k2) { return 6.283185307179586f * ((float)k2 * (1.0f / 16777216.0f)); }

// The per-argument correction bits: bit k of log_fix (cos_fix) set where the host's logf(u1)
// (cosf(angle)) is the neighbour of the rounded double value; bit j of log_any (cos_any) set where any
// of the arguments 16 j .. 16 j + 15 has its bit set. The corrections are rare (0.7% and 1.3% of the
// arguments), so the 128 KiB summaries answer most draws and stay in the L2; only the arguments
// whose 16-block holds a correction read the 2 MiB bitmaps.
struct NoiseFix {
    const uint32_t* log_fix;
    const uint32_t* cos_fix;
    const uint32_t* log_any;
    const uint32_t* cos_any;
    const double* log_tab;   // kNmLogTab doubles
    const double* cos_tab;   // kNmCosTab doubles
};

__host__ __device__ inline bool nm_bit(const uint32_t* bits, uint32_t k) { return (bits[k >> 5] >> (k & 31)) & 1u; }
__host__ __device__ inline bool nm_fix(const uint32_t* any, const uint32_t* bits, uint32_t k) {
    return nm_bit(any, k >> 4) && nm_bit(bits, k);
}

// sqrtf(-2 logf(u1)) as the host's C library gives it
__host__ __device__ inline float nm_radius(const NoiseFix& fx, uint32_t k1) {
    const double d = nm_log_u1(k1, fx.log_tab);
    float l = (float)d;
    if (nm_fix(fx.log_any, fx.log_fix, k1)) l = nm_toward(l, d);
    return __builtin_sqrtf(-2.0f * l);
}
// cosf(6.283185307179586f u2) as the host's C library gives it
__host__ __device__ inline float nm_cosine(const NoiseFix& fx, uint32_t k2) {
    const double d = nm_cos(nm_angle(k2), fx.cos_tab);
    float c = (float)d;
    if (nm_fix(fx.cos_any, fx.cos_fix, k2)) c = nm_toward(c, d);
    return c;
}

}   // namespace ntc_hip
