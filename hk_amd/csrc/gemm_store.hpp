// Output stores of the prefill GEMM kernels.
//
// A wave's 32x32 tile in the v_mfma_*_32x32x* layout has lane l holding row l % 32 of tokens
// 8*(v/4) + 4*(l/32) + v%4 (v < 16). Stored directly, every store instruction writes two 128-byte
// runs of y[token][row] 4 bytes per lane, and the output stores of a large GEMM then cost more
// than a third of the kernel. Transposed through 4 KB of LDS per wave instead, each instruction
// writes 16 bytes per lane, 8 tokens x 128 bytes (measured at 512 tokens: 3072x1024 12.7 -> 9.8
// us, 1024x3072 10.9 -> 9.4 us).
#pragma once

#include "common.hpp"

namespace hkhip {

typedef float gs_v16f __attribute__((ext_vector_type(16)));

// Stores (mode STORE) or adds to (ACCUMULATE) y for rows rw0..rw0+31 and tokens tk0..tk0+31, all
// in range, with y 16-byte aligned and rows a multiple of 4 (of 8 for SILU_MUL). `st` is this
// wave's 4 KB of LDS; `bias` is this lane's row's bias (0 without one). Every lane of the wave
// must call this. SILU_MUL: rows 2i and 2i + 1 are gate and up, y is [n][rows / 2] and gets
// silu(gate) * up.
__device__ __forceinline__ void gemm_store_tile_wide(float *st, const gs_v16f &acc, float bias, float *y,
                                                     uint32_t rows, uint32_t rw0, uint32_t tk0, int mode) {
    const uint32_t lane = __lane_id(), j = lane & 31, h = lane >> 5;
#pragma unroll
    for (int v = 0; v < 16; v++) st[(8 * (v / 4) + 4 * h + (v % 4)) * 32 + j] = acc[v] + bias;
    if (mode == HKHIP_SILU_MUL) {
        // 32 tokens x 16 pairs: lane takes token 16i + lane / 4 and pairs 4q..4q+3 (q = lane % 4).
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t tl = 16 * i + lane / 4, q = lane % 4;
            const float4 a = *reinterpret_cast<const float4 *>(&st[tl * 32 + 8 * q]);
            const float4 b = *reinterpret_cast<const float4 *>(&st[tl * 32 + 8 * q + 4]);
            *reinterpret_cast<float4 *>(y + uint64_t(tk0 + tl) * (rows / 2) + rw0 / 2 + 4 * q) =
                make_float4(silu_mul(a.x, a.y), silu_mul(a.z, a.w), silu_mul(b.x, b.y), silu_mul(b.z, b.w));
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t tl = 8 * i + lane / 8, rr = 4 * (lane % 8);
        float4 vv = *reinterpret_cast<const float4 *>(&st[tl * 32 + rr]);
        float4 *dst = reinterpret_cast<float4 *>(y + uint64_t(tk0 + tl) * rows + rw0 + rr);
        if (mode == HKHIP_ACCUMULATE) {
            const float4 o = *dst;
            vv.x += o.x;
            vv.y += o.y;
            vv.z += o.z;
            vv.w += o.w;
        }
        *dst = vv;
    }
}

// The tile stored lane by lane: rows and tokens past the ends skipped (edge tiles, unaligned y).
__device__ __forceinline__ void gemm_store_tile(const gs_v16f &acc, float bias, float *y, uint32_t rows, uint32_t n,
                                                uint32_t row, uint32_t tk0, int mode) {
    const uint32_t h = __lane_id() >> 5;
    if (mode == HKHIP_SILU_MUL) { // rows even: the gate row's lane (even row) pairs with the next lane's up row
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float g = acc[v] + bias, u = __shfl_xor(g, 1);
            const uint32_t tok = tk0 + 8 * (v / 4) + 4 * h + (v % 4);
            if (row < rows && (row & 1) == 0 && tok < n) y[uint64_t(tok) * (rows / 2) + row / 2] = silu_mul(g, u);
        }
        return;
    }
    if (row >= rows) return;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const uint32_t tok = tk0 + 8 * (v / 4) + 4 * h + (v % 4);
        if (tok < n) {
            float *dst = y + uint64_t(tok) * rows + row;
            if (mode == HKHIP_ACCUMULATE)
                *dst += acc[v] + bias;
            else
                *dst = acc[v] + bias;
        }
    }
}

} // namespace hkhip
