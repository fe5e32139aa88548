// The correction bits of the device's Gaussian draw, built on the host from its own C library, and the
// factors' tables, copied to each device once per process (2 x 2 MiB, their 2 x 128 KiB summaries and 6 KiB of
// tables, one allocation kept until the process ends).
//
// For every argument k of each Box-Muller factor the host compares its C library's logf / cosf
// with the rounded double value of noise_math.hpp; where they differ it checks that the library's
// value is the float neighbour on the side of the double value, and sets bit k. A C library for
// which that rule fails anywhere is reported at init: the device could not reproduce its draws.
#include <math.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "trainer_impl.hpp"

namespace ntc_hip {

namespace {
std::mutex g_mutex;
std::map<int, NoiseFix> g_fix;
}

// The factors' tables (noise_math.hpp): the log bins' reciprocals rc = 1 / c rounded to double and -ln rc from the
// host's long double logarithm, and cos / sin of j 2 pi / 256 from its long double cosine and sine (the quarter points
// exact). The device gets a copy, so both sides evaluate the factors from the same values.
static void nm_fill_tables(double* log_tab, double* cos_tab) {
    for (int i = 0; i < kNmLogBins; i++) {
        long double c = i == 0 ? 1.0L : (i == kNmLogBins - 1 ? 2.0L : 1.0L + ((long double)i + 0.5L) / kNmLogBins);
        if (i >= kNmLogSplit) c *= 0.5L;
        const double rc = (double)(1.0L / c);
        log_tab[2 * i] = rc;
        log_tab[2 * i + 1] = (double)(-logl((long double)rc));
    }
    const long double step = 6.283185307179586476925286766559005768L / kNmCosSteps;
    for (int j = 0; j <= kNmCosSteps; j++) {
        double c = (double)cosl(step * j), sn = (double)sinl(step * j);
        if (j % (kNmCosSteps / 4) == 0) {
            const int q = j / (kNmCosSteps / 4);
            c = (q == 0 || q == 4) ? 1.0 : (q == 2 ? -1.0 : 0.0);
            sn = q == 1 ? 1.0 : (q == 3 ? -1.0 : 0.0);
        }
        cos_tab[2 * j] = c;
        cos_tab[2 * j + 1] = sn;
    }
}

// bit j of the summary = any of the arguments 16 j .. 16 j + 15 has its bit set (half a word of fix)
std::vector<uint32_t> noise_fix_summary(const std::vector<uint32_t>& fix) {
    std::vector<uint32_t> any((fix.size() * 2 + 31) / 32, 0u);
    for (size_t w = 0; w < fix.size(); w++)
        for (size_t h = 0; h < 2; h++) {
            const size_t j = 2 * w + h;
            if ((fix[w] >> (16 * h)) & 0xFFFFu) any[j >> 5] |= 1u << (j & 31);
        }
    return any;
}

bool noise_fix_for_device(int device, NoiseFix& out, std::string& why) {
    std::lock_guard<std::mutex> lock(g_mutex);
    auto it = g_fix.find(device);
    if (it != g_fix.end()) { out = it->second; return true; }
    const uint32_t n = 1u << 24, words = n / 32;
    std::vector<double> ltab(kNmLogTab), ctab(kNmCosTab);
    nm_fill_tables(ltab.data(), ctab.data());
    std::vector<uint32_t> lfix(words, 0u), cfix(words, 0u);
    std::atomic<uint32_t> bad_log{0xFFFFFFFFu}, bad_cos{0xFFFFFFFFu};
    const unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < nt; t++)
        pool.emplace_back([&, t]() {
            const uint32_t w0 = (uint32_t)((uint64_t)words * t / nt), w1 = (uint32_t)((uint64_t)words * (t + 1) / nt);
            for (uint32_t w = w0; w < w1; w++) {
                uint32_t lb = 0, cb = 0;
                for (uint32_t j = 0; j < 32; j++) {
                    const uint32_t k = 32 * w + j;
                    const float lg = logf(nm_u1(k));
                    const double dl = nm_log_u1(k, ltab.data());
                    if ((float)dl != lg) {
                        if (nm_toward((float)dl, dl) != lg) bad_log = k;
                        lb |= 1u << j;
                    }
                    const float cg = cosf(nm_angle(k));
                    const double dc = nm_cos(nm_angle(k), ctab.data());
                    if ((float)dc != cg) {
                        if (nm_toward((float)dc, dc) != cg) bad_cos = k;
                        cb |= 1u << j;
                    }
                }
                lfix[w] = lb; cfix[w] = cb;
            }
        });
    for (auto& th : pool) th.join();
    if (bad_log != 0xFFFFFFFFu || bad_cos != 0xFFFFFFFFu) {
        char buf[256];
        snprintf(buf, sizeof buf, "the host C library's %s differs from the rounded value by more than one float at argument %u; "
                 "the device noise cannot reproduce it", bad_log != 0xFFFFFFFFu ? "logf" : "cosf",
                 bad_log != 0xFFFFFFFFu ? (unsigned)bad_log : (unsigned)bad_cos);
        why = buf;
        return false;
    }
    const std::vector<uint32_t> lany = noise_fix_summary(lfix), cany = noise_fix_summary(cfix);
    const uint32_t swords = (uint32_t)lany.size();
    uint32_t* buf = nullptr;
    // the tables first (8-byte aligned), then the bitmaps and their summaries
    const size_t tab_words = 2 * (size_t)(kNmLogTab + kNmCosTab);
    const size_t total = tab_words + 2 * (size_t)words + 2 * (size_t)swords;
    NTC_CHECK(ntc_hip::ntc_malloc(&buf, total * sizeof(uint32_t)));
    double* lt = reinterpret_cast<double*>(buf);
    double* ct = lt + kNmLogTab;
    uint32_t *l = buf + tab_words, *c = l + words, *la = c + words, *ca = la + swords;
    NTC_CHECK(hipMemcpy(lt, ltab.data(), kNmLogTab * sizeof(double), hipMemcpyHostToDevice));
    NTC_CHECK(hipMemcpy(ct, ctab.data(), kNmCosTab * sizeof(double), hipMemcpyHostToDevice));
    NTC_CHECK(hipMemcpy(l, lfix.data(), (size_t)words * sizeof(uint32_t), hipMemcpyHostToDevice));
    NTC_CHECK(hipMemcpy(c, cfix.data(), (size_t)words * sizeof(uint32_t), hipMemcpyHostToDevice));
    NTC_CHECK(hipMemcpy(la, lany.data(), (size_t)swords * sizeof(uint32_t), hipMemcpyHostToDevice));
    NTC_CHECK(hipMemcpy(ca, cany.data(), (size_t)swords * sizeof(uint32_t), hipMemcpyHostToDevice));
    out = NoiseFix{ l, c, la, ca, lt, ct };
    g_fix[device] = out;
    return true;
}

}   // namespace ntc_hip
