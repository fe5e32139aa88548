// The two factors of the Box-Muller draw (cuda/ntc_noise.h:42-47), evaluated in double precision
// with the same operations on the host and on the device.
//
// The reference draws sqrtf(-2 logf(u1)) * cosf(2 pi u2) with the host C library, u1 = (k1 + 1) / 2^24,
// u2 = k2 / 2^24. Over the 2^24 values of each argument, logf and cosf of glibc differ from the
// correctly rounded result on 122,123 and 217,508 inputs, always by one float, on the side of the
// exact value. Here each factor is computed in double (accurate to a few units in the last place
// of a double), rounded to float, and moved to the float neighbour on the side of the double value
// wherever a per-argument bit (built once on the host from its own C library, 2 MiB per factor)
// says the host differs. The host verifies at set-up that this rule reproduces its C library on
// every argument; the result is the host's draw bit for bit.
//
// Only IEEE operations that round identically on x86-64 and gfx950 are used: +, -, *, /, fma and
// round-to-nearest-even, no library functions.
#pragma once
#ifdef __HIPCC_RTC__   // hipRTC provides the runtime itself and the fixed-width integer types in its own namespace
using __hip_internal::int8_t; using __hip_internal::int16_t; using __hip_internal::int32_t; using __hip_internal::int64_t;
using __hip_internal::uint8_t; using __hip_internal::uint16_t; using __hip_internal::uint32_t; using __hip_internal::uint64_t;
#else
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

namespace ntc_hip {

// ln((k + 1) / 2^24) for k < 2^24: n = k + 1 = 2^e m with m in [sqrt(1/2), sqrt(2)),
// ln m = 2 atanh(s), s = (m - 1) / (m + 1), |s| < 0.172, as an odd series to s^23.
__host__ __device__ inline double nm_log_u1(uint32_t k) {
    const uint64_t n = (uint64_t)k + 1;
    int e = 63 - __builtin_clzll(n);
    double m = (double)n * __builtin_bit_cast(double, (uint64_t)(1023 - e) << 52);   // n 2^-e, exact
    if (m > 1.41421356237309504880) { m *= 0.5; e += 1; }
    const double s = (m - 1.0) / (m + 1.0), s2 = s * s;
    double p = 1.0 / 23.0;
    p = __builtin_fma(p, s2, 1.0 / 21.0); p = __builtin_fma(p, s2, 1.0 / 19.0); p = __builtin_fma(p, s2, 1.0 / 17.0);
    p = __builtin_fma(p, s2, 1.0 / 15.0); p = __builtin_fma(p, s2, 1.0 / 13.0); p = __builtin_fma(p, s2, 1.0 / 11.0);
    p = __builtin_fma(p, s2, 1.0 / 9.0);  p = __builtin_fma(p, s2, 1.0 / 7.0);  p = __builtin_fma(p, s2, 1.0 / 5.0);
    p = __builtin_fma(p, s2, 1.0 / 3.0);
    const double lm = __builtin_fma(2.0 * s, s2 * p, 2.0 * s);
    const double E = (double)(e - 24);
    // ln 2 split so that E ln2_hi is exact
    return __builtin_fma(E, 6.93147180369123816490e-01, __builtin_fma(E, 1.90821492927058770002e-10, lm));
}

// cos(x) for a float x in [0, 2 pi): x = n pi/2 + r with pi/2 in three parts (the first two with
// 33 significant bits, so n pi/2 is subtracted almost exactly), then the Taylor series of cos r
// (to r^18) or sin r (to r^19) on |r| <= pi/4.
__host__ __device__ inline double nm_cos(float x) {
    const double xd = x;
    const double nd = __builtin_rint(xd * 0.63661977236758134308);
    const int n = (int)nd;
    double r = __builtin_fma(-nd, 1.57079632673412561417e+00, xd);
    r = __builtin_fma(-nd, 6.07710050630396597660e-11, r);
    r = __builtin_fma(-nd, 2.02226624879595063154e-21, r);
    const double r2 = r * r;
    double c = 1.0 / 6402373705728000.0;                 // 1/18!
    c = __builtin_fma(c, -r2, 1.0 / 20922789888000.0);   // 1/16!
    c = __builtin_fma(c, -r2, 1.0 / 87178291200.0);      // 1/14!
    c = __builtin_fma(c, -r2, 1.0 / 479001600.0);        // 1/12!
    c = __builtin_fma(c, -r2, 1.0 / 3628800.0);          // 1/10!
    c = __builtin_fma(c, -r2, 1.0 / 40320.0);            // 1/8!
    c = __builtin_fma(c, -r2, 1.0 / 720.0);              // 1/6!
    c = __builtin_fma(c, -r2, 1.0 / 24.0);
    c = __builtin_fma(c, -r2, 0.5);
    c = __builtin_fma(c, -r2, 1.0);
    double s = 1.0 / 121645100408832000.0;               // 1/19!
    s = __builtin_fma(s, -r2, 1.0 / 355687428096000.0);  // 1/17!
    s = __builtin_fma(s, -r2, 1.0 / 1307674368000.0);    // 1/15!
    s = __builtin_fma(s, -r2, 1.0 / 6227020800.0);       // 1/13!
    s = __builtin_fma(s, -r2, 1.0 / 39916800.0);         // 1/11!
    s = __builtin_fma(s, -r2, 1.0 / 362880.0);           // 1/9!
    s = __builtin_fma(s, -r2, 1.0 / 5040.0);             // 1/7!
    s = __builtin_fma(s, -r2, 1.0 / 120.0);
    s = __builtin_fma(s, -r2, 1.0 / 6.0);
    s = __builtin_fma(s * -r2, r, r);
    const double v = (n & 1) ? s : c;
    return ((n + 1) & 2) ? -v : v;                       // n mod 4 = 0: c, 1: -s, 2: -c, 3: s
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
};

__host__ __device__ inline bool nm_bit(const uint32_t* bits, uint32_t k) { return (bits[k >> 5] >> (k & 31)) & 1u; }
__host__ __device__ inline bool nm_fix(const uint32_t* any, const uint32_t* bits, uint32_t k) {
    return nm_bit(any, k >> 4) && nm_bit(bits, k);
}

// sqrtf(-2 logf(u1)) as the host's C library gives it
__host__ __device__ inline float nm_radius(const NoiseFix& fx, uint32_t k1) {
    const double d = nm_log_u1(k1);
    float l = (float)d;
    if (nm_fix(fx.log_any, fx.log_fix, k1)) l = nm_toward(l, d);
    return __builtin_sqrtf(-2.0f * l);
}
// cosf(6.283185307179586f u2) as the host's C library gives it
__host__ __device__ inline float nm_cosine(const NoiseFix& fx, uint32_t k2) {
    const double d = nm_cos(nm_angle(k2));
    float c = (float)d;
    if (nm_fix(fx.cos_any, fx.cos_fix, k2)) c = nm_toward(c, d);
    return c;
}

}   // namespace ntc_hip
