// Small-batch product for Q4_K (2..32 tokens) on the int8 MFMA units.
//
// Between single-token decode and prefill, the weights still dominate the bytes (each is used by
// a handful of tokens), so this kernel streams them like the decode kernels -- every wave loads
// its rows' blocks straight from HBM into registers, two super-blocks in flight -- but
// multiplies them against the tokens on v_mfma_i32_16x16x64_i8 instead of per-token dot
// products, so the per-weight VALU work no longer grows with the token count.
//
// Arithmetic (hk's CPU kernel, src/quant/gemm.zig kernelK 180-236, per row r, token t,
// super-block b):  y += da*(d*I - dmin*J),  I = sum_s sc_s * sum_{k in s} q*a,
// J = sum_s mn_s * bsum32_s, both exact integers:
//  * I: the 6-bit scale is folded into the weights as two int8 planes, sc = 8*sh + sl, each
//    product at most 105 (one packed 16-bit multiply per four weights); the MFMA chain runs the
//    sh plane, the result is multiplied by 8, then the sl plane is added on top.
//  * J: one v_mfma_f32_16x16x32_bf16 over exact bf16 integers: the mins against the tokens'
//    bsum32 = 64*u + v (the activation buffer's k_mb plane), exact in f32 (|J| < 2^22).
//
// Layout. A workgroup owns 16 rows; its KS waves split the super-blocks (KS is picked so that
// the launch has about 2048 waves) and add their partial sums in LDS at the end. Each wave keeps
// PF super-blocks in flight. MFMA roles: A = weights (row = lane % 16), B = activations (token =
// lane % 16); lane group g = lane / 16 supplies k = 16g..16g+15 of each 64-value chunk, so the
// four groups read a token's chunk as one contiguous 64-byte piece and a row's chunk as two
// 16-byte pieces (groups g and g+2 read the same bytes: low and high nibbles are sub-blocks 2c
// and 2c+1 of chunk c). Output lane l holds rows 4*(l/16) + i (i < 4) of token l % 16.

#include "common.hpp"

namespace hkhip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));

struct SkArgs {
    const uint8_t *w;
    uint32_t rows, K, n;
    const int8_t *aqs;  // k_qs [n][K]
    const float *ad;    // k_d [n][K/256]
    const uint8_t *amb; // k_mb [n][K/256] x 32 bytes
    float *y;
    const float *bias;
    int mode;
};

__device__ __forceinline__ uint4 ld16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }

__device__ __forceinline__ uint32_t mul_bytes(uint32_t nib, uint32_t f2) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(us2, nib) * __builtin_bit_cast(us2, f2));
}

// One super-block's operands of this lane: its row's block header and the 16-byte pieces of
// the four chunks, and per token tile the activations, the min-term words and the scale.
template <int NTT> struct SkBuf {
    uint4 hdr;
    uint4 q[4];
    uint4 a[NTT][4];
    uint4 mb[NTT];
    float da[NTT];
};

template <int NTT, int KS, int PF>
__global__ __launch_bounds__(KS * 64) void mmsk_q4k_kernel(SkArgs a) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t g = lane >> 4, p = lane & 15;
    const uint32_t nsb = a.K / 256;
    const uint32_t r0 = blockIdx.x * 16;
    // This wave's super-blocks.
    const uint32_t sb0 = nsb * wave / KS, sb1 = nsb * (wave + 1) / KS;

    const uint32_t row = r0 + p < a.rows ? r0 + p : a.rows - 1;
    const uint8_t *wrow = a.w + uint64_t(row) * nsb * 144;
    uint32_t tokn[NTT]; // token (tile*16 + p), clamped to the last one
#pragma unroll
    for (int tt = 0; tt < NTT; tt++) {
        const uint32_t tok = 16 * tt + p < a.n ? 16 * tt + p : a.n - 1;
        tokn[tt] = tok;
    }

    auto load = [&](SkBuf<NTT> &b, uint32_t sb) {
        const uint8_t *blk = wrow + uint64_t(sb) * 144;
        b.hdr = ld16(blk);
#pragma unroll
        for (int c = 0; c < 4; c++) b.q[c] = ld16(blk + 16 + 32 * c + 16 * (g & 1));
#pragma unroll
        for (int tt = 0; tt < NTT; tt++) {
            const int8_t *ta = a.aqs + uint64_t(tokn[tt]) * a.K + 256 * sb + 16 * g;
#pragma unroll
            for (int c = 0; c < 4; c++) b.a[tt][c] = ld16(ta + 64 * c);
            b.mb[tt] = ld16(a.amb + (uint64_t(tokn[tt]) * nsb + sb) * 32 + 16 * (g & 1));
            b.da[tt] = a.ad[uint64_t(tokn[tt]) * nsb + sb];
        }
        // A buffer's loads stay together and in order behind the previous buffer's.
        __builtin_amdgcn_sched_barrier(0);
    };

    v4f acc[NTT];
#pragma unroll
    for (int tt = 0; tt < NTT; tt++) acc[tt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](const SkBuf<NTT> &b, float keep) {
        const uint4 h = b.hdr;
        const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
        const uint32_t scl = h.y & k1, mnl = h.z & k1;
        const uint32_t sch = (h.w & k2) | (((h.y >> 6) & k3) << 4);
        const uint32_t mnh = ((h.w >> 4) & k2) | (((h.z >> 6) & k3) << 4);
        const float d = f16_bits_to_f32(h.x & 0xFFFF), ndmin = -f16_bits_to_f32(h.x >> 16);
        // Planes of the four chunks: chunk c, lane group g is sub-block 2c + g/2 (low nibbles for
        // g < 2, high for g >= 2).
        v4i ph[4], pl[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t sc = ((c < 2 ? scl : sch) >> (8 * (2 * (c & 1) + (g >> 1)))) & 0xFF;
            const uint32_t fh = (sc >> 3) * 0x00010001u, fl = (sc & 7) * 0x00010001u;
            const uint32_t sh = 4 * (g >> 1);
            const uint32_t w4[4] = {b.q[c].x, b.q[c].y, b.q[c].z, b.q[c].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t nib = (w4[i] >> sh) & 0x0F0F0F0Fu;
                ph[c][i] = int(mul_bytes(nib, fh));
                pl[c][i] = int(mul_bytes(nib, fl));
            }
        }
        // Min-term A operand: the 8 mins as bf16 integers in lane groups 0 and 1, zero in 2, 3.
        v8bf am;
        {
            uint32_t mw[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t src = q < 2 ? mnl : mnh, s = 16 * (q & 1);
                const float e = (float)((src >> s) & 0xFF), o = (float)((src >> (s + 8)) & 0xFF);
                mw[q] = g < 2 ? (__builtin_bit_cast(uint32_t, e) >> 16) | (__builtin_bit_cast(uint32_t, o) & 0xFFFF0000u) : 0u;
            }
            am = __builtin_bit_cast(v8bf, make_uint4(mw[0], mw[1], mw[2], mw[3]));
        }
        // Scales of this lane's output rows 4*(lane/16) + i: from the lanes that loaded them.
        float dr[4], mr[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            dr[i] = __shfl(d, int(4 * g + i));
            mr[i] = __shfl(ndmin, int(4 * g + i));
        }
#pragma unroll
        for (int tt = 0; tt < NTT; tt++) {
            v4i s = {0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < 4; c++)
                s = __builtin_amdgcn_mfma_i32_16x16x64_i8(ph[c], __builtin_bit_cast(v4i, b.a[tt][c]), s, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) s[i] <<= 3;
#pragma unroll
            for (int c = 0; c < 4; c++)
                s = __builtin_amdgcn_mfma_i32_16x16x64_i8(pl[c], __builtin_bit_cast(v4i, b.a[tt][c]), s, 0, 0, 0);
            const uint4 mbw = g < 2 ? b.mb[tt] : make_uint4(0, 0, 0, 0);
            const v4f j = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, __builtin_bit_cast(v8bf, mbw), v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[tt][i] = fmaf(fmaf((float)s[i], dr[i], mr[i] * j[i]), b.da[tt] * keep, acc[tt][i]);
        }
    };

    // PF super-blocks in flight. Every step issues the same loads and runs the same arithmetic
    // (past the wave's range on repeats of its last super-block, scaled by zero): no branch in the
    // loop, so the in-order memory counter covers exactly the buffer about to be used.
    if (sb0 < sb1) {
        SkBuf<NTT> b[PF];
        const uint32_t last = sb1 - 1;
#pragma unroll
        for (int i = 0; i < PF; i++) load(b[i], sb0 + i < last ? sb0 + i : last);
        for (uint32_t sb = sb0; sb <= last; sb += PF) {
#pragma unroll
            for (int i = 0; i < PF; i++) {
                compute(b[i], sb + i <= last ? 1.0f : 0.0f);
                // Keep the refill behind the compute: hoisted above it, its loads would sit in the
                // in-order memory counter ahead of the wait for this buffer.
                __builtin_amdgcn_sched_barrier(0);
                const uint32_t nx = sb + i + PF;
                load(b[i], nx < last ? nx : last);
            }
        }
    }

    // Partial sums of the waves meet in LDS; wave 0 finishes the rows.
    __shared__ v4f part[KS > 1 ? KS - 1 : 1][NTT][64];
    if (wave > 0) {
#pragma unroll
        for (int tt = 0; tt < NTT; tt++) part[wave - 1][tt][lane] = acc[tt];
    }
    if (KS > 1) __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int tt = 0; tt < NTT; tt++) {
#pragma unroll
            for (int w = 0; w < KS - 1; w++) acc[tt] += part[w][tt][lane];
            const uint32_t tok = 16 * tt + p;
            if (tok < a.n) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t r = r0 + 4 * g + i;
                    if (r < a.rows) {
                        float *dst = a.y + uint64_t(tok) * a.rows + r;
                        const float v = acc[tt][i] + (a.bias ? a.bias[r] : 0.0f);
                        if (a.mode == HKHIP_ACCUMULATE)
                            *dst += v;
                        else
                            *dst = v;
                    }
                }
            }
        }
    }
}

} // namespace

bool mmsk_supports(int t, uint32_t rows, uint32_t cols, uint32_t n) {
    return t == HKHIP_Q4_K && cols % 256 == 0 && rows > 0 && n >= 1 && n <= 32;
}

hipError_t launch_mmsk(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n,
                       float *y, const float *bias, int mode, hipStream_t s) {
    if (!mmsk_supports(t, rows, cols, n)) return hipErrorInvalidValue;
    const ActLayout A = act_layout(n, cols);
    SkArgs a{};
    a.w = w;
    a.rows = rows;
    a.K = cols;
    a.n = n;
    a.aqs = reinterpret_cast<const int8_t *>(xq + A.k_qs);
    a.ad = reinterpret_cast<const float *>(xq + A.k_d);
    a.amb = xq + A.k_mb;
    a.y = y;
    a.bias = bias;
    a.mode = mode;
    // K slices: enough waves for ~2048 in the launch, each with at least 4 super-blocks when
    // the matrix has them.
    const uint32_t tiles = (rows + 15) / 16, nsb = cols / 256;
    uint32_t ks = 1;
    while (ks < 8 && tiles * ks * 2 <= 2048 && nsb / (2 * ks) >= 4) ks *= 2;
    const dim3 grid(tiles);
    typedef void (*sk_kernel_t)(SkArgs);
    sk_kernel_t k;
    if (n <= 16)
        k = ks == 1 ? mmsk_q4k_kernel<1, 1, 4> : ks == 2 ? mmsk_q4k_kernel<1, 2, 4> : ks == 4 ? mmsk_q4k_kernel<1, 4, 4> : mmsk_q4k_kernel<1, 8, 4>;
    else
        k = ks == 1 ? mmsk_q4k_kernel<2, 1, 2> : ks == 2 ? mmsk_q4k_kernel<2, 2, 2> : ks == 4 ? mmsk_q4k_kernel<2, 4, 2> : mmsk_q4k_kernel<2, 8, 2>;
    hipLaunchKernelGGL(k, grid, dim3(ks * 64), 0, s, a);
    return hipGetLastError();
}

} // namespace hkhip
