// Activation quantizers (qact), bit-identical to hk's CPU quantizers:
//   A8  per 32 values: d = amax/127, id = 1/d, q = round_half_away(x*id), s = sum q
//       (src/quant/vecdot.zig:134-148 quantizeA8)
//   Q8K per 256 values: max = the value of largest |x| (first one wins), iscale = -127/max,
//       q = min(127, round_half_away(iscale*x)), d = 1/iscale, bsums over 16
//       (src/quant/vecdot.zig:150-180 quantizeQ8K)
// Divisions are correctly rounded (__fdiv_rn) and roundf rounds half away from zero, as Zig's
// @round does; hk's own CUDA/Vulkan paths use round-half-even and differ from its CPU.
#include "common.hpp"

namespace hkhip {

// A8: one thread per value; a 32-lane half-wave owns one block.
__global__ void qact_a8_kernel(const float *__restrict__ x, uint64_t total, int8_t *__restrict__ qs,
                               float *__restrict__ dout, int32_t *__restrict__ sout) {
    uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    float v = i < total ? x[i] : 0.0f;
    float a = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
    float d = __fdiv_rn(a, 127.0f);
    float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    int q = (int)roundf(v * id);
    int s = q;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) s += __shfl_xor(s, off, 32);
    if (i < total) {
        qs[i] = (int8_t)q;
        if ((i & 31) == 0) {
            dout[i / 32] = d;
            sout[i / 32] = s;
        }
    }
}

// Q8K: one wave per 256-value block, four consecutive values per lane.
__global__ void qact_q8k_kernel(const float *__restrict__ x, uint64_t nblocks, int8_t *__restrict__ qs,
                                float *__restrict__ dout, int16_t *__restrict__ bsout) {
    uint32_t lane = threadIdx.x & 63;
    uint64_t b = (uint64_t(blockIdx.x) * blockDim.x + threadIdx.x) / 64;
    if (b >= nblocks) return; // whole waves exit together
    const float4 v4 = reinterpret_cast<const float4 *>(x + b * QK_K)[lane];
    float v[4] = {v4.x, v4.y, v4.z, v4.w};
    // First index of the largest |x| within the lane (strict >, as the reference's scan).
    float amax = 0.0f, mx = 0.0f;
    int idx = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float a = fabsf(v[j]);
        if (a > amax) {
            amax = a;
            mx = v[j];
            idx = int(lane * 4 + j);
        }
    }
    // Across lanes: larger |x| wins, equal |x| goes to the smaller index.
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        float oa = __shfl_xor(amax, off);
        float om = __shfl_xor(mx, off);
        int oi = __shfl_xor(idx, off);
        if (oa > amax || (oa == amax && oi < idx)) {
            amax = oa;
            mx = om;
            idx = oi;
        }
    }
    int8_t q[4];
    float d;
    if (amax == 0.0f) {
        q[0] = q[1] = q[2] = q[3] = 0;
        d = 0.0f;
    } else {
        float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int t = (int)roundf(iscale * v[j]);
            q[j] = (int8_t)(t < 127 ? t : 127);
        }
        d = __fdiv_rn(1.0f, iscale);
    }
    int s = int(q[0]) + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    uint32_t packed = uint32_t(uint8_t(q[0])) | (uint32_t(uint8_t(q[1])) << 8) | (uint32_t(uint8_t(q[2])) << 16) |
                      (uint32_t(uint8_t(q[3])) << 24);
    reinterpret_cast<uint32_t *>(qs + b * QK_K)[lane] = packed;
    if ((lane & 3) == 0) bsout[b * 16 + lane / 4] = (int16_t)s;
    if (lane == 0) dout[b] = d;
}

hipError_t launch_qact(const float *x, uint32_t n, uint32_t k, int kind, uint8_t *xq, hipStream_t s) {
    ActLayout L = act_layout(n, k);
    uint64_t total = uint64_t(n) * k;
    if (total == 0) return hipSuccess;
    if (kind == HKHIP_ACT_A8) {
        uint64_t grid = (total + 255) / 256;
        qact_a8_kernel<<<uint32_t(grid), 256, 0, s>>>(x, total, reinterpret_cast<int8_t *>(xq + L.a8_qs),
                                                      reinterpret_cast<float *>(xq + L.a8_d),
                                                      reinterpret_cast<int32_t *>(xq + L.a8_s));
    } else {
        uint64_t nb = total / QK_K;
        uint64_t grid = (nb + 3) / 4; // 4 waves per workgroup
        qact_q8k_kernel<<<uint32_t(grid), 256, 0, s>>>(x, nb, reinterpret_cast<int8_t *>(xq + L.k_qs),
                                                       reinterpret_cast<float *>(xq + L.k_d),
                                                       reinterpret_cast<int16_t *>(xq + L.k_bs));
    }
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
