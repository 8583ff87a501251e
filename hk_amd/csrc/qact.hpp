// The Q8K activation planes' writer (hk's quantizeQ8K block, src/quant/vecdot.zig:156-180, with
// the engine's extra planes: layout in common.hpp), shared by the quantizer kernels and the kernels
// that quantize their own output (decode attention).
#pragma once
#include "quant.hpp"

namespace hkhip {

// fp32 -> bf16 bits, round to nearest even (finite inputs).
__device__ __forceinline__ uint32_t bf16_bits_rne(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Token-interleaved copies for the small-batch kernel (tiles > 0; layout in common.hpp): token
// t's entries. The padding positions of the last tile are not written: the reader takes the last
// token's entries for them.
struct QactIl {
    uint8_t *qs;
    uint16_t *mb;
    float *d;
    uint32_t tiles, n, nsb;
};

struct Q8KOut {
    int8_t *qs;
    float *d;
    int16_t *bs;
    uint16_t *mb;
    float *db;
    QactIl il;
};
// Block b of the input, quantized by one wave (r: this lane's part).
__device__ __forceinline__ void q8k_out(const Q8KOut &o, uint64_t b, uint32_t lane, const Q8KQ &r) {
    int8_t *qs = o.qs;
    float *dout = o.d, *dbout = o.db;
    int16_t *bsout = o.bs;
    uint16_t *mbout = o.mb;
    const QactIl &il = o.il;
    reinterpret_cast<uint32_t *>(qs + b * QK_K)[lane] = r.packed;
    if ((lane & 3) == 0) bsout[b * 16 + lane / 4] = (int16_t)r.bsum;
    if (lane == 0) dout[b] = r.d;
    // GEMM min-term operand: the sum over the 32 values of sub-block s, bsum32 = 64*u + v
    // (v in [0, 63], u in [-64, 63]), as the exact bf16 integers 64*u and v. The 16-value sums
    // sit in lanes 4g; sub-block s = groups 2s and 2s+1 (lanes 8s and 8s+4).
    const int b32 = r.bsum + __shfl_down(r.bsum, 4);
    const int bv = b32 & 63;
    const uint16_t mu = uint16_t(bf16_bits_rne((float)(b32 - bv))), mv = uint16_t(bf16_bits_rne((float)bv));
    if ((lane & 7) == 0) {
        mbout[b * 16 + lane / 8] = mu;
        mbout[b * 16 + 8 + lane / 8] = mv;
        dbout[b * 8 + lane / 8] = r.d * (float)b32;
    }
    if (il.tiles) {
        const uint32_t b32i = uint32_t(b); // tokens <= SK_MAX_TOKENS: a small index
        const uint32_t t = b32i / il.nsb, sb = b32i - t * il.nsb;
        const uint32_t tile = t / 16, p = t % 16;
        const uint32_t c64 = 4 * sb + lane / 16, g = (lane % 16) / 4;
        uint8_t *e = il.qs + ((uint64_t(c64) * il.tiles + tile) * 64 + 16 * g + p) * 16 + 4 * (lane % 4);
        *reinterpret_cast<uint32_t *>(e) = r.packed;
        const uint64_t mbase = (uint64_t(sb) * il.tiles + tile) * 256; // in uint16: 2 halves x 16 x 8
        if ((lane & 7) == 0) {
            il.mb[mbase + p * 8 + lane / 8] = mu;
            il.mb[mbase + 128 + p * 8 + lane / 8] = mv;
        }
        if (lane == 0) il.d[(uint64_t(sb) * il.tiles + tile) * 16 + p] = r.d;
    }
}

inline Q8KOut q8k_planes(uint8_t *xq, const ActLayout &L, uint32_t n, uint32_t k) {
    return Q8KOut{reinterpret_cast<int8_t *>(xq + L.k_qs), reinterpret_cast<float *>(xq + L.k_d),
                  reinterpret_cast<int16_t *>(xq + L.k_bs), reinterpret_cast<uint16_t *>(xq + L.k_mb),
                  reinterpret_cast<float *>(xq + L.k_db),
                  QactIl{xq + L.k_il, reinterpret_cast<uint16_t *>(xq + L.k_ilmb), reinterpret_cast<float *>(xq + L.k_ild),
                         L.tiles, n, k / QK_K}};
}

} // namespace hkhip
