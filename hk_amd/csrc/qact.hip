// Activation quantizer kernels (qact): f32 [n][k] -> the engine's activation buffer, with the
// block quantizers of quant.hpp (hk's quantizeA8 / quantizeQ8K, src/quant/vecdot.zig:134-180).
#include "quant.hpp"

namespace hkhip {

// A8: one thread per value; a 32-lane half-wave owns one block. dsb (a8_dsb; null when k is
// not a multiple of 256): d * s in three bf16 parts, [k/256][n][3][8].
__global__ void qact_a8_kernel(const float *__restrict__ x, uint64_t total, int8_t *__restrict__ qs,
                               float *__restrict__ dout, int32_t *__restrict__ sout, float *__restrict__ dsout,
                               uint16_t *__restrict__ dsb, uint32_t n, uint32_t kb) {
    const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const A8Q r = quant_a8_halfwave(i < total ? x[i] : 0.0f);
    if (i < total) {
        qs[i] = (int8_t)r.q;
        if ((i & 31) == 0) {
            const uint64_t b = i / 32;
            const float ds = r.d * (float)r.s;
            dout[b] = r.d;
            sout[b] = r.s;
            dsout[b] = ds;
            if (dsb) {
                // hi keeps the leading 8 significant bits, mid the next 8, lo the rest (<= 8).
                const uint32_t t = uint32_t(b / kb), c = uint32_t(b % kb);
                const uint32_t p0 = __builtin_bit_cast(uint32_t, ds) & 0xFFFF0000u;
                const float r1 = ds - __builtin_bit_cast(float, p0);
                const uint32_t p1 = __builtin_bit_cast(uint32_t, r1) & 0xFFFF0000u;
                const uint32_t p2 = __builtin_bit_cast(uint32_t, r1 - __builtin_bit_cast(float, p1));
                uint16_t *o = dsb + ((uint64_t(c / 8) * n + t) * 3) * 8 + c % 8;
                o[0] = uint16_t(p0 >> 16);
                o[8] = uint16_t(p1 >> 16);
                o[16] = uint16_t(p2 >> 16);
            }
        }
    }
}

// Q8K: one wave per 256-value block, four consecutive values per lane.
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

__global__ void qact_q8k_kernel(const float *__restrict__ x, uint64_t nblocks, int8_t *__restrict__ qs,
                                float *__restrict__ dout, int16_t *__restrict__ bsout, uint16_t *__restrict__ mbout,
                                float *__restrict__ dbout, QactIl il) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t b = (uint64_t(blockIdx.x) * blockDim.x + threadIdx.x) / 64;
    if (b >= nblocks) return; // whole waves exit together
    const Q8KQ r = quant_q8k_wave(reinterpret_cast<const float4 *>(x + b * QK_K)[lane], lane);
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

hipError_t launch_qact(const float *x, uint32_t n, uint32_t k, int kind, uint8_t *xq, hipStream_t s) {
    ActLayout L = act_layout(n, k);
    uint64_t total = uint64_t(n) * k;
    if (total == 0) return hipSuccess;
    if (kind == HKHIP_ACT_A8) {
        uint64_t grid = (total + 255) / 256;
        qact_a8_kernel<<<uint32_t(grid), 256, 0, s>>>(x, total, reinterpret_cast<int8_t *>(xq + L.a8_qs),
                                                      reinterpret_cast<float *>(xq + L.a8_d),
                                                      reinterpret_cast<int32_t *>(xq + L.a8_s),
                                                      reinterpret_cast<float *>(xq + L.a8_ds),
                                                      k % QK_K == 0 ? reinterpret_cast<uint16_t *>(xq + L.a8_dsb) : nullptr,
                                                      n, k / 32);
    } else {
        uint64_t nb = total / QK_K;
        uint64_t grid = (nb + 3) / 4; // 4 waves per workgroup
        qact_q8k_kernel<<<uint32_t(grid), 256, 0, s>>>(x, nb, reinterpret_cast<int8_t *>(xq + L.k_qs),
                                                       reinterpret_cast<float *>(xq + L.k_d),
                                                       reinterpret_cast<int16_t *>(xq + L.k_bs),
                                                       reinterpret_cast<uint16_t *>(xq + L.k_mb),
                                                       reinterpret_cast<float *>(xq + L.k_db),
                                                       QactIl{xq + L.k_il, reinterpret_cast<uint16_t *>(xq + L.k_ilmb),
                                                              reinterpret_cast<float *>(xq + L.k_ild), L.tiles, n,
                                                              k / QK_K});
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
