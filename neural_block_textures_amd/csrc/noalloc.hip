// The printed error of the current model (decode_error: mse_of, main.cpp:1764-1788) without any
// allocation at call time, for callers that cannot allocate device memory (a serving or progress-print
// loop that must not synchronize the device through hipMalloc / hipFree). decode_error allocates its
// per-block partial sums on every call; this variant keeps them in `scratch`, one statically sized array
// per GPU, and adds them on the device. Like decode_error it copies a host latent from pageable memory and
// waits on the trainer's stream to read the totals back, so it cannot be captured into a HIP graph.
//
// `scratch` is a device symbol: in host code its name is no device address. Its address on each GPU
// is looked up once (noalloc_scratch_setup, from Trainer::init with that GPU current) and only that
// pointer is handed to kernels. Every call on a GPU shares that GPU's array: calls that overlap on one
// GPU (two host threads, or two trainers' streams) race on it. Nothing needs clearing: every partial
// a call reads was written by the same call.
#include <mutex>

#include "trainer_impl.hpp"

namespace ntc_hip {

// at most this many 256-pixel blocks in the evaluation extent: ew x eh <= 2^24 pixels (4096 x 4096)
constexpr size_t kNoallocBlocks = 65536;
constexpr size_t kNoallocMaxPixels = kNoallocBlocks * 256;
// per block 4 texture sums, then the 4 totals: 65540 x 8 bytes = 512 KiB + 32 bytes per GPU
static __device__ __align__(256) unsigned long long scratch[kNoallocBlocks * 4 + 4];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
unsigned long long* g_ptr[kMaxDevices] = {};
}   // namespace

// once per GPU, with that GPU current: the device address of its `scratch`
bool noalloc_scratch_setup(int device, std::string& why) {
    if (device < 0 || device >= kMaxDevices) { why = "device ordinal outside the library's table"; return false; }
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_ptr[device]) return true;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        why = std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e);
        return false;
    }
    g_ptr[device] = (unsigned long long*)p;
    return true;
}

static unsigned long long* scratch_of(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    return (device >= 0 && device < kMaxDevices) ? g_ptr[device] : nullptr;
}

// the 4 texture totals over nblk blocks' partials (part[b * 4 + t]) into tot[0..3]; one block of
// 256 threads, integer sums (exact, any order)
__global__ void __launch_bounds__(256) k_sse_totals(const unsigned long long* __restrict__ part, size_t nblk,
                                                    unsigned long long* __restrict__ tot) {
    __shared__ unsigned long long red[4][4];
    unsigned long long s[4] = { 0, 0, 0, 0 };
    for (size_t b = threadIdx.x; b < nblk; b += 256)
#pragma unroll
        for (int t = 0; t < 4; t++) s[t] += part[b * 4 + t];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        unsigned long long v = s[t];
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        if (lane == 0) red[wid][t] = v;
    }
    __syncthreads();
    if (threadIdx.x < 4) tot[threadIdx.x] = red[0][threadIdx.x] + red[1][threadIdx.x] + red[2][threadIdx.x] + red[3][threadIdx.x];
}

void decode_error_noalloc_impl(Impl& I, const float* z_host, int ew, int eh, double* tex_mse, double* weighted) {
    if (I.d.nout % 3 != 0) { fprintf(stderr, "ntc_hip backend: decode_error needs RGB textures (nout a multiple of 3)\n"); exit(1); }
    if (ew <= 0 || ew > I.d.W) ew = I.d.W;
    if (eh <= 0 || eh > I.d.H) eh = I.d.H;
    const size_t npx = (size_t)ew * eh, blocks = (npx + 255) / 256;
    if (npx > kNoallocMaxPixels) {
        fprintf(stderr, "ntc_hip backend: decode_error_noalloc evaluates at most %zu pixels (its static scratch); the extent "
                        "%d x %d has %zu (decode_error has no such limit)\n", kNoallocMaxPixels, ew, eh, npx);
        exit(1);
    }
    unsigned long long* sp = scratch_of(I.device);
    if (!sp) { fprintf(stderr, "ntc_hip backend: decode_error_noalloc before the scratch was set up on device %d\n", I.device); exit(1); }
    const float* zsrc = I.zdec;
    if (z_host) {
        NTC_CHECK(hipMemcpyAsync(I.ztmp, z_host, I.nz * sizeof(float), hipMemcpyHostToDevice, I.stream));
        zsrc = I.ztmp;
    }
    launch_decode(I, zsrc);
    launch_u8_sse(I, ew, eh, sp);
    unsigned long long* tot = sp + kNoallocBlocks * 4;
    hipLaunchKernelGGL(k_sse_totals, dim3(1), dim3(256), 0, I.stream, sp, blocks, tot);
    NTC_CHECK(hipGetLastError());
    unsigned long long h[4];
    NTC_CHECK(hipMemcpyAsync(h, tot, sizeof(h), hipMemcpyDeviceToHost, I.stream));
    NTC_CHECK(hipStreamSynchronize(I.stream));
    const int T = I.d.nout / 3;
    const double np = (double)npx;
    double ws = 0.0;
    for (int t = 0; t < T; t++) {
        if (tex_mse) tex_mse[t] = (double)h[t] / (3.0 * np);
        ws += (double)I.d.cw[3 * t] * (double)h[t];
    }
    if (weighted) *weighted = ws / (3.0 * (double)I.d.wsum * np);
}

}   // namespace ntc_hip
