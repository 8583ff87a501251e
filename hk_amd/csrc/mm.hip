// Prefill GEMM (mm): y[t][r] = dot(W[r], xq[t]) for a batch of tokens on the int8 MFMA units.
//
// Integer arithmetic restates src/quant/gemm.zig (kernelLegacy 131-176, kernelK 180-236 with
// the canonical unpack of unpack.zig:29-160): every per-block / per-group integer sum is exact,
// and each block's sum is scaled by its integer scale before the f32 scale update.
//
// Tiling: a workgroup (4 waves) owns 64 tokens x 64 weight rows; each wave one 32 x 32 tile of
// v_mfma_i32_32x32x32_i8 (v_mfma_i32_32x32x16_i8 for Q6_K's 16-weight groups). The K loop walks
// 256 weights at a time: the workgroup stages the activation int8s and the weights, unpacked
// to int8 (nibbles, 6-bit values with the -32 offset folded in, codebook lookups), in LDS.
// MFMA operand A = activations (tokens as M), B = weights (rows as N), so each lane's 16
// results share one weight row and its scales.

#include "common.hpp"

namespace hkhip {

typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int TT = 64;      // tokens per workgroup
constexpr int TR = 64;      // weight rows per workgroup
constexpr int KS = 256;     // weights per K step
constexpr int LDS_STRIDE = KS + 16; // bytes per LDS row (pad against bank conflicts)

struct MmArgs {
    const uint8_t *w;
    const uint16_t *wscale;
    uint32_t rows, cols, n;
    const int8_t *aqs;
    const float *ad;
    const int16_t *abs;
    float *y;
    const float *bias;
    int mode;
};

__device__ __forceinline__ uint4 ld16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }

template <int T>
__global__ __launch_bounds__(256) void mm_kernel(MmArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t sA[TT * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) int8_t sB[TR * LDS_STRIDE];
    __shared__ int sSc[TR][16];  // integer scale per weight group (Q4_K: per 32 in [0..7]; Q6_K: per 16)
    __shared__ int sMn[TR][8];   // Q4_K mins
    __shared__ float sD[TR][8];  // Q4_K: d, dmin; Q6_K: d; legacy: d per block
    __shared__ float sAd[TT][8]; // activation scale: Q8K per token; A8 per token and block
    __shared__ __attribute__((aligned(16))) int16_t sBs[TT][8]; // Q4_K: bsums summed per 32

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t t0 = blockIdx.y * TT, r0 = blockIdx.x * TR;
    const uint32_t wt = wave >> 1, wr = wave & 1; // wave tile: tokens 32*wt.., rows 32*wr..
    const uint32_t K = a.cols;
    constexpr bool kq = (T == HKHIP_Q4_K || T == HKHIP_Q6_K);
    const uint32_t nsteps = (K + KS - 1) / KS;

    float accf[16];
#pragma unroll
    for (int v = 0; v < 16; v++) accf[v] = 0.0f;

    const uint32_t j = lane & 31, khalf = lane >> 5; // MFMA fragment row and k half
    const uint32_t myrow = 32 * wr + j;               // local weight row of this lane's results

    for (uint32_t step = 0; step < nsteps; step++) {
        const uint32_t k0 = step * KS;
        const uint32_t kw = (K - k0 < KS) ? (K - k0) : KS; // weights in this step (multiple of 32)

        // ---- stage activations: 64 tokens x kw bytes, 16 B per thread per pass ----
        for (uint32_t e = tid; e < TT * (KS / 16); e += 256) {
            const uint32_t tt = e / (KS / 16), c = e % (KS / 16);
            uint4 v = make_uint4(0, 0, 0, 0);
            if (t0 + tt < a.n && 16 * c < kw) v = ld16(a.aqs + uint64_t(t0 + tt) * K + k0 + 16 * c);
            *reinterpret_cast<uint4 *>(sA + tt * LDS_STRIDE + 16 * c) = v;
        }
        if (tid < TT) {
            const uint32_t tt = tid;
            const bool ok = t0 + tt < a.n;
            if constexpr (kq) {
                sAd[tt][0] = ok ? a.ad[uint64_t(t0 + tt) * (K / 256) + step] : 0.0f;
                if constexpr (T == HKHIP_Q4_K) {
                    const int16_t *bs = a.abs + uint64_t(t0 + tt) * (K / 16) + 16 * step;
#pragma unroll
                    for (int s = 0; s < 8; s++) sBs[tt][s] = ok ? int16_t(bs[2 * s] + bs[2 * s + 1]) : int16_t(0);
                }
            } else {
#pragma unroll
                for (int b = 0; b < 8; b++)
                    sAd[tt][b] = (ok && 32 * b < kw) ? a.ad[uint64_t(t0 + tt) * (K / 32) + k0 / 32 + b] : 0.0f;
            }
        }

        // ---- stage weights: 64 rows, 4 threads per row ----
        {
            const uint32_t rr = tid >> 2, part = tid & 3;
            const uint32_t grow = r0 + rr;
            const bool ok = grow < a.rows;
            int8_t *dst = sB + rr * LDS_STRIDE;
            if constexpr (T == HKHIP_Q4_K) {
                const uint8_t *blk = a.w + (uint64_t(grow) * (K / 256) + step) * 144;
                uint4 q0 = make_uint4(0, 0, 0, 0), q1 = q0, h = q0;
                if (ok) {
                    q0 = ld16(blk + 16 + 32 * part);
                    q1 = ld16(blk + 32 + 32 * part);
                    h = ld16(blk);
                }
                const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
                uint32_t *lo = reinterpret_cast<uint32_t *>(dst + 64 * part);
                uint32_t *hi = reinterpret_cast<uint32_t *>(dst + 64 * part + 32);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    lo[i] = qw[i] & 0x0F0F0F0Fu;
                    hi[i] = (qw[i] >> 4) & 0x0F0F0F0Fu;
                }
                if (part == 0) {
                    const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
                    const uint32_t s0 = h.y, s1 = h.z, s2 = h.w;
                    const uint32_t mn_hi = ((s2 >> 4) & k2) | (((s1 >> 6) & k3) << 4);
                    const uint32_t mn_lo = s1 & k1;
                    const uint32_t sc_hi = (s2 & k2) | (((s0 >> 6) & k3) << 4);
                    const uint32_t sc_lo = s0 & k1;
#pragma unroll
                    for (int s = 0; s < 4; s++) {
                        sSc[rr][s] = (sc_lo >> (8 * s)) & 0xFF;
                        sSc[rr][4 + s] = (sc_hi >> (8 * s)) & 0xFF;
                        sMn[rr][s] = (mn_lo >> (8 * s)) & 0xFF;
                        sMn[rr][4 + s] = (mn_hi >> (8 * s)) & 0xFF;
                    }
                    sD[rr][0] = f16_bits_to_f32(h.x & 0xFFFF);
                    sD[rr][1] = f16_bits_to_f32(h.x >> 16);
                }
            } else if constexpr (T == HKHIP_Q6_K) {
                const uint32_t n = part >> 1, lc = part & 1;
                const uint8_t *blk = a.w + (uint64_t(grow) * (K / 256) + step) * 208;
                uint4 l0 = make_uint4(0, 0, 0, 0), l1 = l0, hh = l0;
                if (ok) {
                    l0 = ld16(blk + 64 * n + 16 * lc);
                    l1 = ld16(blk + 64 * n + 32 + 16 * lc);
                    hh = ld16(blk + 128 + 32 * n + 16 * lc);
                }
                const uint32_t L0[4] = {l0.x, l0.y, l0.z, l0.w}, L1[4] = {l1.x, l1.y, l1.z, l1.w},
                               H[4] = {hh.x, hh.y, hh.z, hh.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    // 6-bit values minus 32, as signed bytes: (q ^ 0x20) - 0x20 == q - 32 for q < 64.
                    uint32_t q[4];
                    q[0] = (L0[i] & 0x0F0F0F0Fu) | ((H[i] & 0x03030303u) << 4);
                    q[1] = (L1[i] & 0x0F0F0F0Fu) | (((H[i] >> 2) & 0x03030303u) << 4);
                    q[2] = ((L0[i] >> 4) & 0x0F0F0F0Fu) | (((H[i] >> 4) & 0x03030303u) << 4);
                    q[3] = ((L1[i] >> 4) & 0x0F0F0F0Fu) | (((H[i] >> 6) & 0x03030303u) << 4);
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        // per byte: q in [0,63] -> q - 32 in two's complement bytes
                        const uint32_t sgn = q[p] ^ 0x20202020u;         // q - 32 + 32 with bit 5 flipped
                        const uint32_t m = ((sgn >> 5) & 0x01010101u) * 0xE0u; // bit 5 set -> negative
                        const uint32_t val = ok ? ((q[p] & 0x1F1F1F1Fu) | m) : 0u;
                        *reinterpret_cast<uint32_t *>(dst + 128 * n + 32 * p + 16 * lc + 4 * i) = val;
                    }
                }
                if (part == 0) {
                    const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192);
#pragma unroll
                    for (int g = 0; g < 16; g++) sSc[rr][g] = ok ? int(sc[g]) : 0;
                    sD[rr][0] = ok ? f16_bits_to_f32(a.wscale[uint64_t(grow) * (K / 256) + step]) : 0.0f;
                }
            } else {
                // Legacy: 8 blocks of 32 per step; each thread does blocks `part` and `part + 4`.
#pragma unroll
                for (int h2 = 0; h2 < 2; h2++) {
                    const uint32_t b = part + 4 * h2;
                    const bool okb = ok && 32 * b < kw;
                    const uint64_t gb = uint64_t(grow) * (K / 32) + k0 / 32 + b;
                    uint32_t qw[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                    if (okb) {
                        if constexpr (T == HKHIP_Q8_0) {
                            const uint4 x0 = ld16(a.w + gb * 32), x1 = ld16(a.w + gb * 32 + 16);
                            qw[0] = x0.x; qw[1] = x0.y; qw[2] = x0.z; qw[3] = x0.w;
                            qw[4] = x1.x; qw[5] = x1.y; qw[6] = x1.z; qw[7] = x1.w;
                        } else {
                            const uint4 x = ld16(a.w + gb * 16);
                            const uint32_t n4[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                            for (int i = 0; i < 4; i++) {
                                qw[i] = iq4nl_lookup4(n4[i] & 0x0F0F0F0Fu);
                                qw[4 + i] = iq4nl_lookup4((n4[i] >> 4) & 0x0F0F0F0Fu);
                            }
                        }
                    }
                    uint32_t *o = reinterpret_cast<uint32_t *>(dst + 32 * b);
#pragma unroll
                    for (int i = 0; i < 8; i++) o[i] = qw[i];
                    sD[rr][b] = okb ? f16_bits_to_f32(a.wscale[gb]) : 0.0f;
                }
            }
        }
        __syncthreads();

        // ---- MFMA over the step ----
        const int8_t *pa = sA + (32 * wt + j) * LDS_STRIDE;
        const int8_t *pb = sB + myrow * LDS_STRIDE;
        if constexpr (T == HKHIP_Q4_K) {
            int acci[16];
#pragma unroll
            for (int v = 0; v < 16; v++) acci[v] = 0;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const v4i fa = *reinterpret_cast<const v4i *>(pa + 32 * s + 16 * khalf);
                const v4i fb = *reinterpret_cast<const v4i *>(pb + 32 * s + 16 * khalf);
                v16i p = {};
                p = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fb, p, 0, 0, 0);
                const int sc = sSc[myrow][s];
#pragma unroll
                for (int v = 0; v < 16; v++) acci[v] += sc * p[v];
            }
            const float d = sD[myrow][0], dmin = sD[myrow][1];
            int mn[8];
#pragma unroll
            for (int s = 0; s < 8; s++) mn[s] = sMn[myrow][s];
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const uint32_t ti = 32 * wt + 8 * (v / 4) + 4 * khalf + (v % 4);
                const float ad = sAd[ti][0];
                int c = 0;
#pragma unroll
                for (int s = 0; s < 8; s++) c += mn[s] * int(sBs[ti][s]);
                accf[v] = fmaf((float)acci[v], d * ad, accf[v]);
                accf[v] = fmaf((float)c, -(dmin * ad), accf[v]);
            }
        } else if constexpr (T == HKHIP_Q6_K) {
            int acci[16];
#pragma unroll
            for (int v = 0; v < 16; v++) acci[v] = 0;
#pragma unroll
            for (int g = 0; g < 16; g++) {
                const long fa = *reinterpret_cast<const long *>(pa + 16 * g + 8 * khalf);
                const long fb = *reinterpret_cast<const long *>(pb + 16 * g + 8 * khalf);
                v16i p = {};
                p = __builtin_amdgcn_mfma_i32_32x32x16_i8(fa, fb, p, 0, 0, 0);
                const int sc = sSc[myrow][g];
#pragma unroll
                for (int v = 0; v < 16; v++) acci[v] += sc * p[v];
            }
            const float d = sD[myrow][0];
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const uint32_t ti = 32 * wt + 8 * (v / 4) + 4 * khalf + (v % 4);
                accf[v] = fmaf((float)acci[v], d * sAd[ti][0], accf[v]);
            }
        } else {
            const uint32_t nb = kw / 32;
            for (uint32_t b = 0; b < nb; b++) {
                const v4i fa = *reinterpret_cast<const v4i *>(pa + 32 * b + 16 * khalf);
                const v4i fb = *reinterpret_cast<const v4i *>(pb + 32 * b + 16 * khalf);
                v16i p = {};
                p = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fb, p, 0, 0, 0);
                const float d = sD[myrow][b];
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const uint32_t ti = 32 * wt + 8 * (v / 4) + 4 * khalf + (v % 4);
                    accf[v] = fmaf((float)p[v], d * sAd[ti][b], accf[v]);
                }
            }
        }
        __syncthreads();
    }

    // ---- store token-major, with bias ----
    const uint32_t grow = r0 + myrow;
    if (a.mode == HKHIP_SILU_MUL) { // lanes j, j ^ 1 hold rows 2i (gate) and 2i + 1 (up)
        const float b = (a.bias && grow < a.rows) ? a.bias[grow] : 0.0f;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float g = accf[v] + b, u = __shfl_xor(g, 1);
            const uint32_t tok = t0 + 32 * wt + 8 * (v / 4) + 4 * khalf + (v % 4);
            if (grow < a.rows && (grow & 1) == 0 && tok < a.n) a.y[uint64_t(tok) * (a.rows / 2) + grow / 2] = silu_mul(g, u);
        }
        return;
    }
    if (grow < a.rows) {
        const float b = a.bias ? a.bias[grow] : 0.0f;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const uint32_t tok = t0 + 32 * wt + 8 * (v / 4) + 4 * khalf + (v % 4);
            if (tok < a.n) {
                float *dst = a.y + uint64_t(tok) * a.rows + grow;
                if (a.mode == HKHIP_ACCUMULATE)
                    *dst += accf[v] + b;
                else
                    *dst = accf[v] + b;
            }
        }
    }
}

hipError_t launch_mm(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n,
                     float *y, const float *bias, int mode, hipStream_t s) {
    if (rows == 0 || n == 0) return hipSuccess;
    if (fallback_type(t)) return launch_mmvq(t, w, rows, cols, xq, n, y, bias, mode, s); // decode passes of 8
    // Few tokens: the weights dominate, so the kernel that streams them (small-batch MFMA); many:
    // the tiled GEMM.
    if (n >= SK_MIN_TOKENS && mmsk_supports(t, rows, cols, n)) return launch_mmsk(t, w, rows, cols, xq, n, y, bias, mode, s);
    if (mm2_supports(t, rows, cols, n)) return launch_mm2(t, w, rows, cols, xq, n, y, bias, mode, s);
    if (mmx_supports(t, rows, cols, n)) return launch_mmx(t, w, rows, cols, xq, n, y, bias, mode, s);
    // Q4_0..Q5_1 rows that are not whole super-blocks: decode passes of 8 tokens.
    if (legacy32(t) && t != HKHIP_Q8_0 && t != HKHIP_IQ4_NL)
        return launch_mmvq(t, w, rows, cols, xq, n, y, bias, mode, s);
    WLayout W = weight_layout(t, rows, cols);
    ActLayout A = act_layout(n, cols);
    const bool kq = (t == HKHIP_Q4_K || t == HKHIP_Q6_K);
    MmArgs a{};
    a.w = w;
    a.wscale = reinterpret_cast<const uint16_t *>(w + W.scale_off);
    a.rows = rows;
    a.cols = cols;
    a.n = n;
    a.aqs = reinterpret_cast<const int8_t *>(xq + (kq ? A.k_qs : A.a8_qs));
    a.ad = reinterpret_cast<const float *>(xq + (kq ? A.k_d : A.a8_d));
    a.abs = reinterpret_cast<const int16_t *>(xq + A.k_bs);
    a.y = y;
    a.bias = bias;
    a.mode = mode;
    dim3 grid((rows + TR - 1) / TR, (n + TT - 1) / TT);
    switch (t) {
    case HKHIP_Q4_K: mm_kernel<HKHIP_Q4_K><<<grid, 256, 0, s>>>(a); break;
    case HKHIP_Q6_K: mm_kernel<HKHIP_Q6_K><<<grid, 256, 0, s>>>(a); break;
    case HKHIP_Q8_0: mm_kernel<HKHIP_Q8_0><<<grid, 256, 0, s>>>(a); break;
    case HKHIP_IQ4_NL: mm_kernel<HKHIP_IQ4_NL><<<grid, 256, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

} // namespace hkhip
