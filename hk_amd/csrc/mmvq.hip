// Decode matvec (mmvq): y[t][r] = dot(W[r], xq[t]) for 1..8 tokens, straight from the quantized
// weights. Integer parts follow src/quant/vecdot.zig exactly (dotQ8_0 235-250, dotIQ4NL 369-384,
// k4Block/dotQ4K 482-522, dotQ6K 533-570); only the order of the f32 scale accumulation differs.
//
// Mapping: a row is owned by `lpr` lanes of one wave (64, or fewer when the row has fewer work
// units, so short rows pack several rows per wave). A unit is the slice of a row one lane
// handles per step, chosen so every lane issues 16-byte loads:
//   Q4_K   a quarter super-block: 32 B of nibbles (two sub-blocks of 32) + the 16-B header
//   Q6_K   a quarter super-block: 16 B of each of ql-low, ql-high, qh (64 weights, 4 groups)
//   Q8_0   one block: 32 B of int8
//   IQ4_NL one block: 16 B of nibbles, looked up in the codebook with byte permutes
// Products use sdot4 (v_dot4_i32_i8); the lane partials are reduced with cross-lane shuffles.
// Activations are read through the L1/L2 caches; they are a few KB and shared by every row.
#include "common.hpp"

namespace hkhip {

struct MvArgs {
    const uint8_t *w;
    const uint16_t *wscale; // scale plane (Q8_0, IQ4_NL, Q6_K)
    uint32_t rows, cols;
    const int8_t *aqs;  // [n][cols]
    const float *ad;    // [n][cols/32] (A8) or [n][cols/256] (Q8K)
    const int16_t *abs; // [n][cols/16] (Q8K)
    float *y;
    const float *bias;
    int mode;
    int lpr_log2;
};

__device__ __forceinline__ uint4 ld16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }

template <int T, int NT>
__global__ __launch_bounds__(256) void mmvq_kernel(MvArgs a) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t lpr = 1u << a.lpr_log2;
    const uint32_t sub = lane >> a.lpr_log2, ul = lane & (lpr - 1);
    const uint32_t row = (blockIdx.x * 4 + wave) * (64u >> a.lpr_log2) + sub;
    const bool active = row < a.rows;
    const uint32_t K = a.cols;

    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.0f;

    if constexpr (T == HKHIP_Q4_K) {
        const uint32_t nsb = K / 256, U = nsb * 4;
        const uint8_t *wr = a.w + uint64_t(row) * nsb * 144;
        float corr[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) corr[t] = 0.0f;
        for (uint32_t u = ul; active && u < U; u += lpr) {
            const uint32_t sb = u >> 2, c = u & 3;
            const uint8_t *blk = wr + sb * 144;
            const uint4 h = ld16(blk);
            const uint4 q0 = ld16(blk + 16 + 32 * c), q1 = ld16(blk + 32 + 32 * c);
            // scalesMinsK4 word unpack (vecdot.zig:461-474), then the pair of sub-blocks 2c, 2c+1.
            const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
            const uint32_t s0 = h.y, s1 = h.z, s2 = h.w;
            const uint32_t mn_hi = ((s2 >> 4) & k2) | (((s1 >> 6) & k3) << 4);
            const uint32_t mn_lo = s1 & k1;
            const uint32_t sc_hi = (s2 & k2) | (((s0 >> 6) & k3) << 4);
            const uint32_t sc_lo = s0 & k1;
            const uint32_t sh = 16 * (c & 1);
            const uint32_t scw = ((c < 2) ? sc_lo : sc_hi) >> sh, mnw = ((c < 2) ? mn_lo : mn_hi) >> sh;
            const int sc0 = scw & 0xFF, sc1 = (scw >> 8) & 0xFF, mn0 = mnw & 0xFF, mn1 = (mnw >> 8) & 0xFF;
            const float d = f16_bits_to_f32(h.x & 0xFFFF), dmin = f16_bits_to_f32(h.x >> 16);
            const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const int8_t *aq = a.aqs + uint64_t(t) * K + sb * 256 + 64 * c;
                const uint4 a0 = ld16(aq), a1 = ld16(aq + 16), a2 = ld16(aq + 32), a3 = ld16(aq + 48);
                const uint32_t aw[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                                         a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
                int slo = 0, shi = 0;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    slo = sdot4(qw[i] & 0x0F0F0F0Fu, aw[i], slo);
                    shi = sdot4((qw[i] >> 4) & 0x0F0F0F0Fu, aw[8 + i], shi);
                }
                const uint2 bsw = *reinterpret_cast<const uint2 *>(a.abs + uint64_t(t) * (K / 16) + sb * 16 + 4 * c);
                const int b0 = int16_t(bsw.x & 0xFFFF), b1 = int16_t(bsw.x >> 16);
                const int b2 = int16_t(bsw.y & 0xFFFF), b3 = int16_t(bsw.y >> 16);
                const int isum = slo * sc0 + shi * sc1;
                const int csum = mn0 * (b0 + b1) + mn1 * (b2 + b3);
                const float ad = a.ad[uint64_t(t) * nsb + sb];
                acc[t] = fmaf((float)isum, d * ad, acc[t]);
                corr[t] = fmaf((float)csum, dmin * ad, corr[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] -= corr[t];
    } else if constexpr (T == HKHIP_Q6_K) {
        const uint32_t nsb = K / 256, U = nsb * 4;
        const uint8_t *wr = a.w + uint64_t(row) * nsb * 208;
        const uint16_t *dr = a.wscale + uint64_t(row) * nsb;
        for (uint32_t u = ul; active && u < U; u += lpr) {
            const uint32_t sb = u >> 2, n = (u >> 1) & 1, lc = u & 1;
            const uint8_t *blk = wr + sb * 208;
            const uint4 l0 = ld16(blk + 64 * n + 16 * lc), l1 = ld16(blk + 64 * n + 32 + 16 * lc);
            const uint4 hh = ld16(blk + 128 + 32 * n + 16 * lc);
            const uint2 scv = *reinterpret_cast<const uint2 *>(blk + 192 + 8 * n);
            const float d = f16_bits_to_f32(dr[sb]);
            const int sc[4] = {int8_t(scv.x >> (8 * lc)), int8_t(scv.x >> (8 * lc + 16)), int8_t(scv.y >> (8 * lc)),
                               int8_t(scv.y >> (8 * lc + 16))};
            const uint32_t L0[4] = {l0.x, l0.y, l0.z, l0.w}, L1[4] = {l1.x, l1.y, l1.z, l1.w},
                           H[4] = {hh.x, hh.y, hh.z, hh.w};
            uint32_t qv[4][4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                qv[0][i] = (L0[i] & 0x0F0F0F0Fu) | ((H[i] & 0x03030303u) << 4);
                qv[1][i] = (L1[i] & 0x0F0F0F0Fu) | (((H[i] >> 2) & 0x03030303u) << 4);
                qv[2][i] = ((L0[i] >> 4) & 0x0F0F0F0Fu) | (((H[i] >> 4) & 0x03030303u) << 4);
                qv[3][i] = ((L1[i] >> 4) & 0x0F0F0F0Fu) | (((H[i] >> 6) & 0x03030303u) << 4);
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const int8_t *aq = a.aqs + uint64_t(t) * K + sb * 256 + 128 * n + 16 * lc;
                const uint4 bsv = ld16(a.abs + uint64_t(t) * (K / 16) + sb * 16 + 8 * n);
                const uint32_t bw[4] = {bsv.x, bsv.y, bsv.z, bsv.w};
                int isum = 0, bias = 0;
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const uint4 av = ld16(aq + 32 * p);
                    int s = sdot4(qv[p][0], av.x, 0);
                    s = sdot4(qv[p][1], av.y, s);
                    s = sdot4(qv[p][2], av.z, s);
                    s = sdot4(qv[p][3], av.w, s);
                    isum += s * sc[p];
                    bias += sc[p] * int(int16_t(bw[p] >> (16 * lc)));
                }
                const float ad = a.ad[uint64_t(t) * nsb + sb];
                acc[t] = fmaf((float)(isum - 32 * bias), d * ad, acc[t]);
            }
        }
    } else { // Q8_0 and IQ4_NL against A8
        const uint32_t U = K / 32;
        const uint64_t rb = uint64_t(row) * U;
        for (uint32_t u = ul; active && u < U; u += lpr) {
            uint32_t qw[8];
            if constexpr (T == HKHIP_Q8_0) {
                const uint4 q0 = ld16(a.w + (rb + u) * 32), q1 = ld16(a.w + (rb + u) * 32 + 16);
                qw[0] = q0.x; qw[1] = q0.y; qw[2] = q0.z; qw[3] = q0.w;
                qw[4] = q1.x; qw[5] = q1.y; qw[6] = q1.z; qw[7] = q1.w;
            } else {
                const uint4 q = ld16(a.w + (rb + u) * 16);
                const uint32_t n4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    qw[i] = iq4nl_lookup4(n4[i] & 0x0F0F0F0Fu);
                    qw[4 + i] = iq4nl_lookup4((n4[i] >> 4) & 0x0F0F0F0Fu);
                }
            }
            const float d = f16_bits_to_f32(a.wscale[rb + u]);
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const int8_t *aq = a.aqs + uint64_t(t) * K + 32 * u;
                const uint4 a0 = ld16(aq), a1 = ld16(aq + 16);
                int s = sdot4(qw[0], a0.x, 0);
                s = sdot4(qw[1], a0.y, s);
                s = sdot4(qw[2], a0.z, s);
                s = sdot4(qw[3], a0.w, s);
                s = sdot4(qw[4], a1.x, s);
                s = sdot4(qw[5], a1.y, s);
                s = sdot4(qw[6], a1.z, s);
                s = sdot4(qw[7], a1.w, s);
                acc[t] = fmaf((float)s, d * a.ad[uint64_t(t) * U + u], acc[t]);
            }
        }
    }

    // Reduce the lane partials of each row group.
#pragma unroll
    for (int t = 0; t < NT; t++) {
        for (uint32_t off = lpr >> 1; off > 0; off >>= 1) acc[t] += __shfl_xor(acc[t], off);
    }
    if (active && ul == 0) {
        const float b = a.bias ? a.bias[row] : 0.0f;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float *dst = a.y + uint64_t(t) * a.rows + row;
            if (a.mode == HKHIP_ACCUMULATE)
                *dst += acc[t] + b;
            else
                *dst = acc[t] + b;
        }
    }
}

template <int T>
static hipError_t launch_fmt(const MvArgs &a, uint32_t n, uint32_t grid, hipStream_t s) {
    switch (n) {
    case 1: mmvq_kernel<T, 1><<<grid, 256, 0, s>>>(a); break;
    case 2: mmvq_kernel<T, 2><<<grid, 256, 0, s>>>(a); break;
    case 3: mmvq_kernel<T, 3><<<grid, 256, 0, s>>>(a); break;
    case 4: mmvq_kernel<T, 4><<<grid, 256, 0, s>>>(a); break;
    case 5: mmvq_kernel<T, 5><<<grid, 256, 0, s>>>(a); break;
    case 6: mmvq_kernel<T, 6><<<grid, 256, 0, s>>>(a); break;
    case 7: mmvq_kernel<T, 7><<<grid, 256, 0, s>>>(a); break;
    case 8: mmvq_kernel<T, 8><<<grid, 256, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_mmvq(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n,
                       float *y, const float *bias, int mode, hipStream_t s) {
    if (n < 1 || n > 8) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    WLayout W = weight_layout(t, rows, cols);
    ActLayout A = act_layout(n, cols);
    const bool kq = (t == HKHIP_Q4_K || t == HKHIP_Q6_K);
    MvArgs a{};
    a.w = w;
    a.wscale = reinterpret_cast<const uint16_t *>(w + W.scale_off);
    a.rows = rows;
    a.cols = cols;
    a.aqs = reinterpret_cast<const int8_t *>(xq + (kq ? A.k_qs : A.a8_qs));
    a.ad = reinterpret_cast<const float *>(xq + (kq ? A.k_d : A.a8_d));
    a.abs = reinterpret_cast<const int16_t *>(xq + A.k_bs);
    a.y = y;
    a.bias = bias;
    a.mode = mode;
    const uint32_t units = kq ? cols / 64 : cols / 32;
    int lg = 0;
    while ((1u << lg) < units && lg < 6) lg++;
    a.lpr_log2 = lg;
    const uint32_t rows_per_block = 4u * (64u >> lg);
    const uint32_t grid = (rows + rows_per_block - 1) / rows_per_block;
    switch (t) {
    case HKHIP_Q4_K: return launch_fmt<HKHIP_Q4_K>(a, n, grid, s);
    case HKHIP_Q6_K: return launch_fmt<HKHIP_Q6_K>(a, n, grid, s);
    case HKHIP_Q8_0: return launch_fmt<HKHIP_Q8_0>(a, n, grid, s);
    case HKHIP_IQ4_NL: return launch_fmt<HKHIP_IQ4_NL>(a, n, grid, s);
    default: return hipErrorInvalidValue;
    }
}

} // namespace hkhip
