// Activation quantizers shared by the qact kernels and the matvec prologue, bit-identical to
// hk's CPU quantizers:
//   A8  per 32 values: d = amax/127, id = 1/d, q = round_half_away(x*id), s = sum q
//       (src/quant/vecdot.zig:134-148 quantizeA8)
//   Q8K per 256 values: max = the value of largest |x| (the first one wins), iscale = -127/max,
//       q = min(127, round_half_away(iscale*x)), d = 1/iscale, bsums over 16
//       (src/quant/vecdot.zig:150-180 quantizeQ8K)
// Divisions are correctly rounded (__fdiv_rn) and roundf rounds half away from zero, as Zig's
// @round does; hk's own CUDA/Vulkan paths use round-half-even and differ from its CPU.
//
// Reductions run on DPP lane moves inside each row of 16 lanes and v_readlane across rows, so a
// block costs a few dozen cycles instead of a chain of LDS-routed shuffles.
#pragma once

#include "common.hpp"

namespace hkhip {

// DPP controls (row = 16 lanes).
constexpr int DPP_XOR1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <-> 7-i within 8
constexpr int DPP_MIRROR = 0x140;      // lane i <-> 15-i within 16
constexpr int DPP_ROR8 = 0x128;        // lane i <-> i ^ 8 within 16 (rotate by 8)

template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL> __device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Max over each row of 16 lanes (every lane of the row gets it).
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    return fmaxf(v, dpp_f<DPP_MIRROR>(v));
}
__device__ __forceinline__ int row_sum(int v) {
    v += dpp_i<DPP_XOR1>(v);
    v += dpp_i<DPP_XOR2>(v);
    v += dpp_i<DPP_HALF_MIRROR>(v);
    return v + dpp_i<DPP_MIRROR>(v);
}

struct A8Q {
    int q;   // this lane's quantized value
    float d; // block scale
    int s;   // block sum of q
};

// One A8 block per 32-lane half-wave (lanes 0-31 and 32-63 are two blocks), one value per lane.
// All 64 lanes must be active.
__device__ __forceinline__ A8Q quant_a8_halfwave(float v) {
    const uint32_t lane = __lane_id();
    const float rm = row_max(fabsf(v));
    const float a = lane < 32 ? fmaxf(readlane_f(rm, 0), readlane_f(rm, 16))
                              : fmaxf(readlane_f(rm, 32), readlane_f(rm, 48));
    A8Q r;
    r.d = __fdiv_rn(a, 127.0f);
    const float id = r.d != 0.0f ? __fdiv_rn(1.0f, r.d) : 0.0f;
    r.q = (int)roundf(v * id);
    const int rs = row_sum(r.q);
    r.s = lane < 32 ? __builtin_amdgcn_readlane(rs, 0) + __builtin_amdgcn_readlane(rs, 16)
                    : __builtin_amdgcn_readlane(rs, 32) + __builtin_amdgcn_readlane(rs, 48);
    return r;
}

struct Q8KQ {
    uint32_t packed; // this lane's four quantized values (bytes, lowest first)
    float d;         // block scale
    int bsum;        // sum over this lane's group of 16 (four lanes)
};

// One Q8K block per 64-lane wave, four consecutive values per lane (lane l holds 4l..4l+3).
// All 64 lanes must be active.
__device__ __forceinline__ Q8KQ quant_q8k_wave(float4 v4, uint32_t lane) {
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    const float lmax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    const float rm = row_max(lmax);
    const float amax = fmaxf(fmaxf(readlane_f(rm, 0), readlane_f(rm, 16)), fmaxf(readlane_f(rm, 32), readlane_f(rm, 48)));
    // The signed value of the first element reaching amax (strict > scan in the reference).
    float first = 0.0f;
    bool hit = false;
#pragma unroll
    for (int j = 3; j >= 0; j--) {
        if (fabsf(v[j]) == amax) {
            first = v[j];
            hit = true;
        }
    }
    const uint64_t mask = __ballot(hit);
    Q8KQ r;
    int q[4] = {0, 0, 0, 0};
    if (amax == 0.0f || mask == 0) {
        r.d = 0.0f;
    } else {
        const float mx = readlane_f(first, __builtin_ctzll(mask));
        const float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int t = (int)roundf(iscale * v[j]);
            q[j] = t < 127 ? t : 127;
        }
        r.d = __fdiv_rn(1.0f, iscale);
    }
    int s = q[0] + q[1] + q[2] + q[3];
    s += dpp_i<DPP_XOR1>(s);
    s += dpp_i<DPP_XOR2>(s);
    r.bsum = s;
    r.packed = uint32_t(uint8_t(q[0])) | (uint32_t(uint8_t(q[1])) << 8) | (uint32_t(uint8_t(q[2])) << 16) |
               (uint32_t(uint8_t(q[3])) << 24);
    (void)lane;
    return r;
}

} // namespace hkhip
