// Activation quantizer kernels (qact): f32 [n][k] -> the engine's activation buffer, with the
// block quantizers of quant.hpp (hk's quantizeA8 / quantizeQ8K, src/quant/vecdot.zig:134-180).
#include "qact.hpp"

namespace hkhip {

// The A8 planes (dsb, a8_dsb: null when k is not a multiple of 256: d * s in three bf16 parts,
// [k/256][n][3][8]).
struct A8Out {
    int8_t *qs;
    float *d;
    int32_t *s;
    float *ds;
    uint16_t *dsb;
    uint32_t n, kb; // tokens, blocks per row
};
// Value i of the input (block i / 32); the lane of each block's first value writes the block's data.
__device__ __forceinline__ void a8_out(const A8Out &o, uint64_t i, const A8Q &r) {
    o.qs[i] = (int8_t)r.q;
    if ((i & 31) == 0) {
        const uint64_t b = i / 32;
        const float ds = r.d * (float)r.s;
        o.d[b] = r.d;
        o.s[b] = r.s;
        o.ds[b] = ds;
        if (o.dsb) {
            // hi keeps the leading 8 significant bits, mid the next 8, lo the rest (<= 8).
            const uint32_t t = uint32_t(b / o.kb), c = uint32_t(b % o.kb);
            const uint32_t p0 = __builtin_bit_cast(uint32_t, ds) & 0xFFFF0000u;
            const float r1 = ds - __builtin_bit_cast(float, p0);
            const uint32_t p1 = __builtin_bit_cast(uint32_t, r1) & 0xFFFF0000u;
            const uint32_t p2 = __builtin_bit_cast(uint32_t, r1 - __builtin_bit_cast(float, p1));
            uint16_t *q = o.dsb + ((uint64_t(c / 8) * o.n + t) * 3) * 8 + c % 8;
            q[0] = uint16_t(p0 >> 16);
            q[8] = uint16_t(p1 >> 16);
            q[16] = uint16_t(p2 >> 16);
        }
    }
}

// A8: one thread per value; a 32-lane half-wave owns one block.
__global__ void qact_a8_kernel(const float *__restrict__ x, uint64_t total, A8Out o) {
    const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const A8Q r = quant_a8_halfwave(i < total ? x[i] : 0.0f);
    if (i < total) a8_out(o, i, r);
}

// Q8K: one wave per 256-value block, four consecutive values per lane (q8k_out: qact.hpp).
__global__ void qact_q8k_kernel(const float *__restrict__ x, uint64_t nblocks, Q8KOut o) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t b = (uint64_t(blockIdx.x) * blockDim.x + threadIdx.x) / 64;
    if (b >= nblocks) return; // whole waves exit together
    q8k_out(o, b, lane, quant_q8k_wave(reinterpret_cast<const float4 *>(x + b * QK_K)[lane], lane));
}

// The quantizers with the RMS norm folded in, workgroups of 256 threads over the token rows (k
// values each): value i = (x[i] * inv) * norm[i], inv = 1 / sqrt(mean(x^2) + eps) (ops.zig:10-29;
// the sum of squares in the order of the standalone RMS norm kernel: 256 strided partial sums,
// then the workgroup reduction). Then each block is quantized as qact_a8_kernel / qact_q8k_kernel
// quantize it.
struct RowIn {
    const float *x;
    const float *norm; // or null
    float eps;
    uint32_t k;
};
__device__ __forceinline__ float row_value(const RowIn &in, const float *xr, float inv, uint32_t i) {
    if (in.norm) return (xr[i] * inv) * in.norm[i];
    return xr[i];
}
__device__ __forceinline__ float row_inv(const RowIn &in, const float *xr) {
    __shared__ float red[4];
    if (!in.norm) return 1.0f;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < in.k; i += 256) ss = fmaf(xr[i], xr[i], ss);
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = red[0] + red[1] + red[2] + red[3];
    return __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, float(in.k)) + in.eps));
}

// Grid (token row, piece of the row): a workgroup quantizes QACT_ROW_PIECE values of its row (the
// norm's factor from the whole row, summed the same way in every workgroup), so a long row spreads
// over several CUs instead of one workgroup looping over it.
constexpr uint32_t QACT_ROW_PIECE = 1024;

__global__ __launch_bounds__(256) void qact_a8_row_kernel(RowIn in, A8Out o) {
    const uint32_t t = blockIdx.x;
    const float *xr = in.x + uint64_t(t) * in.k;
    const float inv = row_inv(in, xr);
    const uint32_t i1 = min(in.k, QACT_ROW_PIECE * (blockIdx.y + 1));
    for (uint32_t i0 = QACT_ROW_PIECE * blockIdx.y; i0 < i1; i0 += 256) { // k is a multiple of 32: whole half-waves
        const uint32_t i = i0 + threadIdx.x;
        const bool live = i < i1;
        const A8Q r = quant_a8_halfwave(live ? row_value(in, xr, inv, i) : 0.0f);
        if (live) a8_out(o, uint64_t(t) * in.k + i, r);
    }
}

// Four consecutive values i..i+3 of a row (i a multiple of 4), with 16-byte loads.
__device__ __forceinline__ float4 row_values4(const RowIn &in, const float *xr, float inv, uint32_t i) {
    const float4 x = *reinterpret_cast<const float4 *>(xr + i);
    if (!in.norm) return x;
    const float4 w = *reinterpret_cast<const float4 *>(in.norm + i);
    return make_float4((x.x * inv) * w.x, (x.y * inv) * w.y, (x.z * inv) * w.z, (x.w * inv) * w.w);
}

__global__ __launch_bounds__(256) void qact_q8k_row_kernel(RowIn in, Q8KOut o) {
    const uint32_t t = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const float *xr = in.x + uint64_t(t) * in.k;
    const float inv = row_inv(in, xr);
    const uint32_t nsb = in.k / QK_K, sb = blockIdx.y * (QACT_ROW_PIECE / QK_K) + w; // one block per wave
    if (sb < nsb)
        q8k_out(o, uint64_t(t) * nsb + sb, lane, quant_q8k_wave(row_values4(in, xr, inv, sb * QK_K + 4 * lane), lane));
}

// The norm case for rows of up to QACT_NORM_LDS values, workgroups of (row, piece of 1024 values): the 16-byte load
// f = 256 i + thread of the row is value 4 f.. of block 4 i + wave, lanes in value order, which is
// exactly what the wave quantizing that block wants, so every value and its norm weight are loaded
// once, up front, into registers (all loads in flight together), the sum of squares is reduced with
// one barrier, and each wave quantizes the block of its workgroup's piece from its registers. (Norm
// weights loaded inside the block loop, and the row staged through LDS, put a dependent global
// round trip per block behind two barriers: 6.2-7.6 us per launch at 8-512 rows; one workgroup per
// row, each wave quantizing its four blocks in turn: 8 sequences per Llama-3-8B pass 2.668 vs 2.529
// ms with the row split four ways.)
constexpr uint32_t QACT_NORM_LDS = 8192;
__global__ __launch_bounds__(256) void qact_q8k_norm_row_kernel(RowIn in, Q8KOut o) {
    constexpr int IT = QACT_NORM_LDS / QK_K / 4; // blocks per wave at most
    __shared__ float red[4];
    const uint32_t t = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t nsb = in.k / QK_K;
    const float4 *xr4 = reinterpret_cast<const float4 *>(in.x + uint64_t(t) * in.k);
    const float4 *g4 = reinterpret_cast<const float4 *>(in.norm);
    float4 x[IT], g[IT];
#pragma unroll
    for (int it = 0; it < IT; it++)
        if (w + 4 * it < nsb) x[it] = xr4[(w + 4 * it) * 64 + lane];
#pragma unroll
    for (int it = 0; it < IT; it++)
        if (uint32_t(it) == blockIdx.y && w + 4 * it < nsb) g[it] = g4[(w + 4 * it) * 64 + lane];
    float ss = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; it++) {
        if (w + 4 * it < nsb) {
            ss = fmaf(x[it].x, x[it].x, ss);
            ss = fmaf(x[it].y, x[it].y, ss);
            ss = fmaf(x[it].z, x[it].z, ss);
            ss = fmaf(x[it].w, x[it].w, ss);
        }
    }
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    if (lane == 0) red[w] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, float(in.k)) + in.eps));
    // Workgroup (row, piece) quantizes blocks 4 piece .. 4 piece + 3 (one per wave; its loads hold
    // them), every workgroup of the row summing the squares of the whole row in the same order.
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const uint32_t sb = w + 4 * it;
        if (uint32_t(it) == blockIdx.y && sb < nsb) {
            const float4 v = make_float4((x[it].x * inv) * g[it].x, (x[it].y * inv) * g[it].y,
                                         (x[it].z * inv) * g[it].z, (x[it].w * inv) * g[it].w);
            q8k_out(o, uint64_t(t) * nsb + sb, lane, quant_q8k_wave(v, lane));
        }
    }
}

static A8Out a8_planes(uint8_t *xq, const ActLayout &L, uint32_t n, uint32_t k) {
    return A8Out{reinterpret_cast<int8_t *>(xq + L.a8_qs), reinterpret_cast<float *>(xq + L.a8_d),
                 reinterpret_cast<int32_t *>(xq + L.a8_s), reinterpret_cast<float *>(xq + L.a8_ds),
                 k % QK_K == 0 ? reinterpret_cast<uint16_t *>(xq + L.a8_dsb) : nullptr, n, k / 32};
}
hipError_t launch_qact(const float *x, uint32_t n, uint32_t k, int kind, uint8_t *xq, hipStream_t s) {
    ActLayout L = act_layout(n, k);
    uint64_t total = uint64_t(n) * k;
    if (total == 0) return hipSuccess;
    if (kind == HKHIP_ACT_A8) {
        uint64_t grid = (total + 255) / 256;
        qact_a8_kernel<<<uint32_t(grid), 256, 0, s>>>(x, total, a8_planes(xq, L, n, k));
    } else {
        uint64_t nb = total / QK_K;
        uint64_t grid = (nb + 3) / 4; // 4 waves per workgroup
        qact_q8k_kernel<<<uint32_t(grid), 256, 0, s>>>(x, nb, q8k_planes(xq, L, n, k));
    }
    return hipGetLastError();
}

hipError_t launch_qact_row(const float *x, uint32_t n, uint32_t k, int kind, uint8_t *xq, const float *norm, float eps,
                           hipStream_t s) {
    if (n == 0 || k == 0) return hipSuccess;
    if (k % 32 || (kind != HKHIP_ACT_A8 && k % QK_K)) return hipErrorInvalidValue;
    const ActLayout L = act_layout(n, k);
    const RowIn in{x, norm, eps, k};
    const dim3 grid(n, (k + QACT_ROW_PIECE - 1) / QACT_ROW_PIECE);
    if (kind == HKHIP_ACT_A8)
        qact_a8_row_kernel<<<grid, 256, 0, s>>>(in, a8_planes(xq, L, n, k));
    else if (norm && k <= QACT_NORM_LDS)
        qact_q8k_norm_row_kernel<<<dim3(n, (k / QK_K + 3) / 4), 256, 0, s>>>(in, q8k_planes(xq, L, n, k));
    else
        qact_q8k_row_kernel<<<grid, 256, 0, s>>>(in, q8k_planes(xq, L, n, k));
    return hipGetLastError();
}

// Packs one kind of the device buffer into hk's block structs (40-byte A8, 292-byte Q8K).
__global__ void act_pack_kernel(const uint8_t *__restrict__ xq, ActLayout L, uint64_t nblocks, int kind,
                                uint8_t *__restrict__ out) {
    uint64_t b = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    if (kind == HKHIP_ACT_A8) {
        uint8_t *o = out + b * 40;
        *reinterpret_cast<float *>(o) = reinterpret_cast<const float *>(xq + L.a8_d)[b];
        *reinterpret_cast<int32_t *>(o + 4) = reinterpret_cast<const int32_t *>(xq + L.a8_s)[b];
        for (int j = 0; j < 32; j++) o[8 + j] = xq[L.a8_qs + b * 32 + j];
    } else {
        uint8_t *o = out + b * 292;
        float d = reinterpret_cast<const float *>(xq + L.k_d)[b];
        const uint8_t *dp = reinterpret_cast<const uint8_t *>(&d);
        for (int j = 0; j < 4; j++) o[j] = dp[j];
        for (int j = 0; j < 256; j++) o[4 + j] = xq[L.k_qs + b * 256 + j];
        const uint8_t *bs = xq + L.k_bs + b * 32;
        for (int j = 0; j < 32; j++) o[260 + j] = bs[j];
    }
}

hipError_t launch_act_pack(const uint8_t *xq, uint32_t n, uint32_t k, int kind, uint8_t *out, hipStream_t s) {
    ActLayout L = act_layout(n, k);
    uint64_t nb = uint64_t(n) * k / (kind == HKHIP_ACT_A8 ? 32 : QK_K);
    if (nb == 0) return hipSuccess;
    act_pack_kernel<<<uint32_t((nb + 255) / 256), 256, 0, s>>>(xq, L, nb, kind, out);
    return hipGetLastError();
}

} // namespace hkhip
