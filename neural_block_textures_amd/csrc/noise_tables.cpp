// The two factor tables of the Gaussian draw, built on the host from the C library and copied to
// each device once per process.
//
// The reference draws sqrtf(-2 logf(u1)) * cosf(2 pi u2) with the host C library (cuda/ntc_noise.h:
// 42-47), and u1, u2 take only 2^24 values each. glibc's logf and cosf are not correctly rounded
// on a fraction of those inputs, so no device-side evaluation can promise the host's bits; the
// tables make the device's draw equal the host's by construction, whatever C library the caller
// links. 2 x 64 MiB per device, kept until the process ends.
#include <math.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <thread>
#include <vector>

#include "trainer_impl.hpp"

namespace ntc_hip {

namespace {
std::mutex g_mutex;
std::map<int, NoiseTables> g_tables;
}

NoiseTables noise_tables_for_device(int device) {
    std::lock_guard<std::mutex> lock(g_mutex);
    auto it = g_tables.find(device);
    if (it != g_tables.end()) return it->second;
    const size_t n = (size_t)1 << 24;
    std::vector<float> rad(n), cosv(n);
    const unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < nt; t++)
        pool.emplace_back([&, t]() {
            const size_t k0 = n * t / nt, k1 = n * (t + 1) / nt;
            for (size_t k = k0; k < k1; k++) {
                const float u1 = (float)(k + 1) * (1.0f / 16777216.0f);   // (0, 1]
                const float u2 = (float)k * (1.0f / 16777216.0f);         // [0, 1)
                rad[k] = sqrtf(-2.0f * logf(u1));
                cosv[k] = cosf(6.283185307179586f * u2);
            }
        });
    for (auto& th : pool) th.join();
    NoiseTables T{};
    float *r = nullptr, *c = nullptr;
    NTC_CHECK(hipMalloc(&r, n * sizeof(float)));
    NTC_CHECK(hipMalloc(&c, n * sizeof(float)));
    NTC_CHECK(hipMemcpy(r, rad.data(), n * sizeof(float), hipMemcpyHostToDevice));
    NTC_CHECK(hipMemcpy(c, cosv.data(), n * sizeof(float), hipMemcpyHostToDevice));
    T.rad = r; T.cosv = c;
    g_tables[device] = T;
    return T;
}

}   // namespace ntc_hip
