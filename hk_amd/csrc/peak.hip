// Measured peaks of this GPU, for the benchmark to quote beside the published ones: the dense
// int8 MFMA rate (v_mfma_i32_32x32x32_i8 chains on every SIMD) and the HBM streaming-read rate.
// Built into its own library (libhkpeak.so); not part of the engine's C ABI.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));

// Four independent accumulator chains per wave (enough to cover the MFMA latency); operands are
// pseudo-random bytes, since the MFMA units' power (and so their sustained clock) depends on the
// data.
__global__ __launch_bounds__(256) void mfma_i8_kernel(uint32_t iters, int *out) {
    uint32_t s = 0x9E3779B9u * (threadIdx.x + 1) ^ (blockIdx.x * 0x85EBCA6Bu);
    auto next = [&]() {
        s ^= s << 13;
        s ^= s >> 17;
        s ^= s << 5;
        return int(s);
    };
    const v4i a0 = {next(), next(), next(), next()}, a1 = {next(), next(), next(), next()};
    const v4i b0 = {next(), next(), next(), next()}, b1 = {next(), next(), next(), next()};
    v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (uint32_t i = 0; i < iters; i++) {
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b0, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b1, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, c3, 0, 0, 0);
    }
    int r = 0;
#pragma unroll
    for (int v = 0; v < 16; v++) r ^= c0[v] + c1[v] + c2[v] + c3[v];
    out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

// Streaming read: each thread sums 16-byte words grid-strided over the buffer.
__global__ __launch_bounds__(256) void read_kernel(const uint4 *p, uint64_t n16, uint32_t *out) {
    uint32_t acc = 0;
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const uint4 v = p[i];
        acc ^= v.x + v.y + v.z + v.w;
    }
    out[blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

int cu_count() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    return n;
}

// Median rate (amount per second, `amount` the ops or bytes of one run) of up to 16 timed runs.
template <typename L> double median_rate(int reps, double amount, L launch) {
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0;
    launch(); // warm-up
    const int nrep = reps < 1 ? 1 : reps > 16 ? 16 : reps;
    double t[16];
    bool ok = true;
    for (int r = 0; r < nrep && ok; r++) {
        ok = hipEventRecord(e0, nullptr) == hipSuccess;
        launch();
        ok = ok && hipEventRecord(e1, nullptr) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
        float ms = 0.0f;
        ok = ok && hipEventElapsedTime(&ms, e0, e1) == hipSuccess && ms > 0.0f;
        t[r] = ok ? amount / (double(ms) * 1e-3) : 0.0;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (!ok || hipGetLastError() != hipSuccess) return -1.0;
    for (int i = 1; i < nrep; i++) // insertion sort
        for (int k = i; k > 0 && t[k] < t[k - 1]; k--) {
            const double x = t[k];
            t[k] = t[k - 1];
            t[k - 1] = x;
        }
    return t[nrep / 2];
}

} // namespace

extern "C" {

// Dense int8 MFMA rate in TOPS (2 ops per multiply-add): median of `reps` launches of about
// 5 ms, four waves per SIMD. Negative on a HIP error.
double hkpeak_mfma_i8_tops(int reps) {
    const int cus = cu_count();
    if (cus <= 0) return -1.0;
    const uint32_t blocks = uint32_t(cus) * 4, threads = 256, iters = 20000;
    int *out = nullptr;
    if (hipMalloc(&out, size_t(blocks) * threads * sizeof(int)) != hipSuccess) return -1.0;
    const double ops = double(blocks) * (threads / 64) * iters * 4.0 * 2.0 * 32 * 32 * 32;
    const double r = median_rate(reps, ops, [&] { mfma_i8_kernel<<<blocks, threads>>>(iters, out); });
    (void)hipFree(out);
    return r < 0 ? r : r / 1e12;
}

// Streaming-read rate of a `bytes` buffer in GB/s (make it larger than the 256 MB Infinity Cache
// for an HBM figure): median of `reps` launches. Negative on a HIP error.
double hkpeak_read_gbs(uint64_t bytes, int reps) {
    const int cus = cu_count();
    if (cus <= 0 || bytes < 16) return -1.0;
    const uint64_t n16 = bytes / 16;
    const uint32_t blocks = uint32_t(cus) * 8, threads = 256;
    uint4 *buf = nullptr;
    uint32_t *out = nullptr;
    if (hipMalloc(&buf, n16 * 16) != hipSuccess) return -1.0;
    double r = -1.0;
    if (hipMalloc(&out, size_t(blocks) * threads * 4) == hipSuccess && hipMemset(buf, 1, n16 * 16) == hipSuccess)
        r = median_rate(reps, double(n16 * 16), [&] { read_kernel<<<blocks, threads>>>(buf, n16, out); });
    (void)hipFree(out);
    (void)hipFree(buf);
    return r < 0 ? r : r / 1e9;
}

} // extern "C"
