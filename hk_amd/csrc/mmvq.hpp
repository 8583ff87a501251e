#pragma once
// Kernels of the decode matvec (mmvq): y[t][r] = dot(W[r], x[t]) for 1..8 tokens, straight from the quantized
// weights. Integer parts follow src/quant/vecdot.zig exactly (dotQ8_0 235-250, dotIQ4NL 369-384,
// k4Block/dotQ4K 482-522, dotQ6K 533-570); only the order of the f32 scale accumulation differs.
//
// One launch computes up to four matrices that read the same input (q/k/v, gate/up), the way
// matmul.runParts fuses them on the CPU (src/engine/matmul.zig:96-144).
//
// Work unit: a slice of a row that one lane reads with 16-byte loads:
//   Q4_K   a quarter super-block: 32 B of nibbles (two sub-blocks of 32) + the 16-B header
//   Q6_K   a quarter super-block: 16 B of each of ql-low, ql-high, qh (64 weights, 4 groups)
//   Q8_0   one block: 32 B of int8
//   IQ4_NL one block: 16 B of nibbles, looked up in the codebook with byte permutes
//   Q4_0, Q4_1, Q5_0, Q5_1  one block: 16 B of nibbles + side-plane d (m, fifth bits)
// Products use sdot4 (v_dot4_i32_i8); lane partials are reduced with DPP lane moves.
//
// Two kernels:
//  * mmvr_kernel (the decode path): lane l of a wave owns units l, l+64, ... of every row and
//    holds their activations in registers; a wave streams whole rows (one-token launches deal
//    them to the waves in turn, a step's rows at a time), so each activation register serves
//    every row. Used when the activations fit the registers
//    (rows of up to 256-512 units, depending on format and token count).
//  * mmvq_kernel (everything else): a row is shared by 2^k lanes that step through it, and the
//    activations stay in LDS.
// Both are persistent (about one wave set per SIMD) with double-buffered weight loads, and both
// quantize an f32 input themselves, once per workgroup, with the qact arithmetic (quant.hpp), so
// that a decode step needs no separate quantization launch.
#include "quant.hpp"

namespace hkhip {

constexpr int MV_PARTS = 4;
constexpr uint32_t MV_LDS_MAX = 160 * 1024; // LDS per workgroup on gfx950

struct MvPart {
    const uint8_t *w;
    const uint16_t *ws; // scale plane (Q8_0, IQ4_NL, Q6_K)
    float *y;
    const float *bias;
    uint32_t rows;
    uint32_t gstart; // first row group of this part (parts start on a group boundary)
};

struct MvArgs {
    MvPart p[MV_PARTS];
    uint32_t nparts, ngroups, K;
    const float *x;    // f32 input [NT][K], quantized in the prologue; or null
    const int8_t *gqs; // pre-quantized input (engine activation buffer) when x is null
    const float *gd;
    const int16_t *gbs;
    int mode;
    int lpr_log2;
    uint32_t ntok; // tokens actually present (register kernel; at most its NT)
    // Register kernel on an f32 input: when set, the input is first RMS-normalized per token,
    // x * (1 / sqrt(mean(x^2) + eps)) * norm (ops.zig:10-29 rmsNorm), then quantized.
    const float *norm;
    float eps;
    // Register kernel: rows dealt to the row groups in turn, one step's rows (R * (64 >> LG)) at a
    // time, instead of a contiguous range per group (a step's loads then cover one contiguous
    // span of the matrix across the whole grid).
    int interleave;
};

// Chunks of 1024 inputs a wave of the register kernel stages in one pass (its prefetch depth).
__host__ __device__ constexpr int mvr_pb(bool kq, int nt, int c, int nw) {
    return (kq ? 4 : 2) * nt * c / nw < 1 ? 1 : (kq ? 4 : 2) * nt * c / nw > 4 ? 4 : (kq ? 4 : 2) * nt * c / nw;
}

__device__ __forceinline__ uint4 ldw(const void *p) { return *reinterpret_cast<const uint4 *>(p); }

// LDS layout for NT tokens of K: qs [NT][K] i8 | bsums [NT][K/16] i16 (Q8K) | d [NT][K/blk] f32.
// Within a token, 16-byte chunks are permuted inside aligned groups of four (K-quants; two for
// A8) so that the chunks consecutive lanes read in one instruction fall in different banks.
__host__ __device__ inline uint32_t mv_lds_bytes(int nt, uint32_t K, bool kq) {
    return nt * K + (kq ? nt * K / 8 : 0) + nt * (K / (kq ? 256 : 32)) * 4;
}

template <uint32_t MASK> __device__ __forceinline__ uint32_t swz(uint32_t c) {
    return c ^ (((c >> 3) ^ (c >> 4)) & MASK);
}

// Activations staged in LDS.
struct ActL {
    const int8_t *qs;
    const int16_t *bs;
    const float *d;
    uint32_t K;
};

// Where one lane's row lives.
struct RowRef {
    const uint8_t *w;   // first byte of the row in the quant plane
    const uint16_t *ws; // first scale of the row in the scale (side) plane
    const uint16_t *wm; // Q4_1 / Q5_1: the row's offsets m
    const uint32_t *wh; // Q5_0 / Q5_1: the row's fifth-bit words
};

// ---------------------------------------------------------------------------------------------
// Per-format pieces. units(K): work units per row. lds_chunk / bs_index: LDS position of the
// natural 16-B activation chunk / bsum within a token. W: one unit of weights, AU: the matching
// activations. dot: one unit against one token.
// ---------------------------------------------------------------------------------------------

template <int T> struct MvFmt;

// Q4_K and Q5_K (hk's file blocks, 144 / 176 B; Q5_K adds qh[32] before qs).
template <int T> struct MvK4 {
    static constexpr bool kq = true;
    static constexpr bool five = (T == HKHIP_Q5_K);
    static constexpr uint32_t BB = five ? 176 : 144, QO = five ? 48 : 16; // block bytes, qs offset
    __device__ static uint32_t units(uint32_t K) { return K / 64; }
    __device__ static uint32_t lds_chunk(uint32_t c) { return swz<3>(c); }
    __device__ static uint32_t bs_index(uint32_t g) { return g; }
    struct W {
        uint4 h, q0, q1, x0, x1; // x: Q5_K's qh[32]
    };
    struct AU {
        uint32_t q[16];
        int b01, b23;
        float d;
    };
    __device__ static RowRef row(const uint8_t *w, const uint16_t *, uint32_t r, uint32_t K) {
        return RowRef{w + uint64_t(r) * (K / 256) * BB, nullptr};
    }
    // Offset in the token of the j-th 16-value chunk of unit u (natural order; chunks ascend in j).
    __device__ static uint32_t chunk_off(uint32_t u, uint32_t j) { return 64 * u + 16 * j; }
    __device__ static AU make(const uint32_t *q, const int *bs, float d) {
        AU a;
#pragma unroll
        for (int i = 0; i < 16; i++) a.q[i] = q[i];
        a.b01 = bs[0] + bs[1];
        a.b23 = bs[2] + bs[3];
        a.d = d;
        return a;
    }
    __device__ static W load(const RowRef &R, uint32_t u) {
        const uint8_t *blk = R.w + (u >> 2) * BB;
        W w;
        w.h = ldw(blk);
        w.q0 = ldw(blk + QO + 32 * (u & 3));
        w.q1 = ldw(blk + QO + 16 + 32 * (u & 3));
        if constexpr (five) {
            w.x0 = ldw(blk + 16);
            w.x1 = ldw(blk + 32);
        }
        return w;
    }
    // Unit u = quarter q of super-block sb: activation bytes 64q..64q+63, bsums 4q..4q+3.
    __device__ static AU act(const ActL &A, uint32_t t, uint32_t u) {
        const uint32_t base = t * (A.K / 16);
        AU a;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint4 v = ldw(A.qs + 16 * (base + swz<3>(4 * u + j)));
            a.q[4 * j] = v.x; a.q[4 * j + 1] = v.y; a.q[4 * j + 2] = v.z; a.q[4 * j + 3] = v.w;
        }
        const uint2 b = *reinterpret_cast<const uint2 *>(A.bs + base + 4 * u);
        a.b01 = int(int16_t(b.x & 0xFFFF)) + int(int16_t(b.x >> 16));
        a.b23 = int(int16_t(b.y & 0xFFFF)) + int(int16_t(b.y >> 16));
        a.d = A.d[t * (A.K / 256) + (u >> 2)];
        return a;
    }
    // Weight-side work of a unit, done once for all tokens: the two sub-block scales and mins
    // (scalesMinsK4 word unpack, vecdot.zig:461-474) and the unpacked nibbles.
    struct P {
        uint32_t lo[8], hi[8];
        int sc0, sc1, mn0, mn1;
        float d, dmin;
    };
    __device__ static P prep(const W &w, uint32_t u) {
        const uint32_t q = u & 3;
        const uint4 h = w.h;
        const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
        const uint32_t sh = 16 * (q & 1);
        uint32_t scw, mnw;
        if (q < 2) {
            scw = (h.y & k1) >> sh;
            mnw = (h.z & k1) >> sh;
        } else {
            scw = ((h.w & k2) | (((h.y >> 6) & k3) << 4)) >> sh;
            mnw = (((h.w >> 4) & k2) | (((h.z >> 6) & k3) << 4)) >> sh;
        }
        P p;
        p.sc0 = scw & 0xFF; p.sc1 = (scw >> 8) & 0xFF; p.mn0 = mnw & 0xFF; p.mn1 = (mnw >> 8) & 0xFF;
        const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        const uint32_t xw[8] = {w.x0.x, w.x0.y, w.x0.z, w.x0.w, w.x1.x, w.x1.y, w.x1.z, w.x1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            p.lo[i] = qw[i] & 0x0F0F0F0Fu;
            p.hi[i] = (qw[i] >> 4) & 0x0F0F0F0Fu;
            if constexpr (five) { // k4Block has_high: bits 2q / 2q+1 of qh[l] (vecdot.zig:492-495)
                p.lo[i] |= ((xw[i] >> (2 * q)) & 0x01010101u) << 4;
                p.hi[i] |= ((xw[i] >> (2 * q + 1)) & 0x01010101u) << 4;
            }
        }
        p.d = f16_bits_to_f32(h.x & 0xFFFF);
        p.dmin = f16_bits_to_f32(h.x >> 16);
        return p;
    }
    // One token: sub-blocks 2q and 2q+1 of the super-block (k4Block, vecdot.zig:482-522).
    __device__ static void dotp(const P &p, const AU &a, float &acc, float &corr) {
        int slo = 0, shi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            slo = sdot4(p.lo[i], a.q[i], slo);
            shi = sdot4(p.hi[i], a.q[8 + i], shi);
        }
        acc = fmaf((float)(slo * p.sc0 + shi * p.sc1), p.d * a.d, acc);
        corr = fmaf((float)(p.mn0 * a.b01 + p.mn1 * a.b23), p.dmin * a.d, corr);
    }
    __device__ static void dot(const W &w, uint32_t u, const AU &a, float &acc, float &corr) {
        dotp(prep(w, u), a, acc, corr);
    }
};
template <> struct MvFmt<HKHIP_Q4_K> : MvK4<HKHIP_Q4_K> {};
template <> struct MvFmt<HKHIP_Q5_K> : MvK4<HKHIP_Q5_K> {};

// IQ4_XS (dotIQ4XS, vecdot.zig:572-597): a unit is sub-blocks 2q, 2q+1 of a super-block: 32 B of
// codebook indices (quant plane, 128 B per block) and the block's 8-B header (side plane: d,
// scales_h, scales_l); against Q8K, so the activation side is Q4_K's.
template <> struct MvFmt<HKHIP_IQ4_XS> : MvK4<HKHIP_Q4_K> {
    struct W {
        uint4 q0, q1;
        uint2 h;
    };
    __device__ static RowRef row(const uint8_t *w, const uint16_t *ws, uint32_t r, uint32_t K) {
        return RowRef{w + uint64_t(r) * (K / 256) * 128, ws + uint64_t(r) * (K / 256) * 4};
    }
    __device__ static W load(const RowRef &R, uint32_t u) {
        const uint8_t *q = R.w + (u >> 2) * 128 + 32 * (u & 3);
        W w;
        w.q0 = ldw(q);
        w.q1 = ldw(q + 16);
        w.h = *reinterpret_cast<const uint2 *>(R.ws + (u >> 2) * 4);
        return w;
    }
    struct P {
        uint32_t q[16];
        int ls0, ls1;
        float d;
    };
    __device__ static P prep(const W &w, uint32_t u) {
        const uint32_t q = u & 3;
        P p;
        const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p.q[8 * s + i] = iq4nl_lookup4(qw[4 * s + i] & 0x0F0F0F0Fu);
                p.q[8 * s + 4 + i] = iq4nl_lookup4((qw[4 * s + i] >> 4) & 0x0F0F0F0Fu);
            }
        // Sub-block scale: low 4 bits from scales_l (byte q: sub-block 2q low nibble, 2q+1 high),
        // high 2 bits from scales_h, minus 32.
        const uint32_t sl = (w.h.y >> (8 * q)) & 0xFF, shb = (w.h.x >> (16 + 4 * q)) & 0xF;
        p.ls0 = int((sl & 0xF) | ((shb & 3) << 4)) - 32;
        p.ls1 = int((sl >> 4) | ((shb >> 2) << 4)) - 32;
        p.d = f16_bits_to_f32(w.h.x & 0xFFFF);
        return p;
    }
    __device__ static void dotp(const P &p, const AU &a, float &acc, float &) {
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s0 = sdot4(p.q[i], a.q[i], s0);
            s1 = sdot4(p.q[8 + i], a.q[8 + i], s1);
        }
        acc = fmaf((float)(s0 * p.ls0 + s1 * p.ls1), p.d * a.d, acc);
    }
    __device__ static void dot(const W &w, uint32_t u, const AU &a, float &acc, float &corr) {
        dotp(prep(w, u), a, acc, corr);
    }
};

template <> struct MvFmt<HKHIP_Q6_K> {
    static constexpr bool kq = true;
    __device__ static uint32_t units(uint32_t K) { return K / 64; }
    // Unit-major within a super-block: the 64 bytes (and 4 bsums) one unit reads are contiguous.
    // Natural chunk m (values 16m..16m+15) is segment p = (m >> 1) & 3 of unit (n = m >> 3,
    // lc = m & 1), unit index 2n + lc.
    __device__ static uint32_t unit_major(uint32_t c) {
        const uint32_t m = c & 15;
        return (c & ~15u) + 4 * (2 * (m >> 3) + (m & 1)) + ((m >> 1) & 3);
    }
    __device__ static uint32_t lds_chunk(uint32_t c) { return swz<3>(unit_major(c)); }
    __device__ static uint32_t bs_index(uint32_t g) { return unit_major(g); }
    struct W {
        uint4 l0, l1, hh;
        uint2 sc;
        uint32_t d;
    };
    struct AU {
        uint32_t q[16];
        int bs[4];
        float d;
    };
    __device__ static RowRef row(const uint8_t *w, const uint16_t *ws, uint32_t r, uint32_t K) {
        return RowRef{w + uint64_t(r) * (K / 256) * 208, ws + uint64_t(r) * (K / 256)};
    }
    __device__ static uint32_t chunk_off(uint32_t u, uint32_t j) {
        return 256 * (u >> 2) + 128 * ((u >> 1) & 1) + 16 * (u & 1) + 32 * j;
    }
    __device__ static AU make(const uint32_t *q, const int *bs, float d) {
        AU a;
#pragma unroll
        for (int i = 0; i < 16; i++) a.q[i] = q[i];
#pragma unroll
        for (int i = 0; i < 4; i++) a.bs[i] = bs[i];
        a.d = d;
        return a;
    }
    __device__ static W load(const RowRef &R, uint32_t u) {
        const uint32_t n = (u >> 1) & 1, lc = u & 1;
        const uint8_t *blk = R.w + (u >> 2) * 208;
        W w;
        w.l0 = ldw(blk + 64 * n + 16 * lc);
        w.l1 = ldw(blk + 64 * n + 32 + 16 * lc);
        w.hh = ldw(blk + 128 + 32 * n + 16 * lc);
        w.sc = *reinterpret_cast<const uint2 *>(blk + 192 + 8 * n);
        w.d = R.ws[u >> 2];
        return w;
    }
    // Unit u = (sb, n, lc): activations 128n + 32p + 16lc + i (p < 4, i < 16), groups 8n + 2p + lc.
    __device__ static AU act(const ActL &A, uint32_t t, uint32_t u) {
        const uint32_t base = t * (A.K / 16);
        AU a;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint4 v = ldw(A.qs + 16 * (base + swz<3>(4 * u + p)));
            a.q[4 * p] = v.x; a.q[4 * p + 1] = v.y; a.q[4 * p + 2] = v.z; a.q[4 * p + 3] = v.w;
        }
        const uint2 b = *reinterpret_cast<const uint2 *>(A.bs + base + 4 * u);
        a.bs[0] = int16_t(b.x & 0xFFFF);
        a.bs[1] = int16_t(b.x >> 16);
        a.bs[2] = int16_t(b.y & 0xFFFF);
        a.bs[3] = int16_t(b.y >> 16);
        a.d = A.d[t * (A.K / 256) + (u >> 2)];
        return a;
    }
    // Weight-side work of a unit: the 6-bit values of its 4 groups of 16 (stored as q, the -32
    // goes through bsums) and their scales.
    struct P {
        uint32_t q[16];
        int sc[4];
        float d;
    };
    __device__ static P prep(const W &w, uint32_t u) {
        const uint32_t lc = u & 1;
        P p;
        p.sc[0] = int8_t(w.sc.x >> (8 * lc));
        p.sc[1] = int8_t(w.sc.x >> (8 * lc + 16));
        p.sc[2] = int8_t(w.sc.y >> (8 * lc));
        p.sc[3] = int8_t(w.sc.y >> (8 * lc + 16));
        const uint32_t L0[4] = {w.l0.x, w.l0.y, w.l0.z, w.l0.w};
        const uint32_t L1[4] = {w.l1.x, w.l1.y, w.l1.z, w.l1.w};
        const uint32_t H[4] = {w.hh.x, w.hh.y, w.hh.z, w.hh.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            p.q[i] = (L0[i] & 0x0F0F0F0Fu) | ((H[i] & 0x03030303u) << 4);
            p.q[4 + i] = (L1[i] & 0x0F0F0F0Fu) | (((H[i] >> 2) & 0x03030303u) << 4);
            p.q[8 + i] = ((L0[i] >> 4) & 0x0F0F0F0Fu) | (((H[i] >> 4) & 0x03030303u) << 4);
            p.q[12 + i] = ((L1[i] >> 4) & 0x0F0F0F0Fu) | (((H[i] >> 6) & 0x03030303u) << 4);
        }
        p.d = f16_bits_to_f32(w.d);
        return p;
    }
    // One token (dotQ6K, vecdot.zig:533-570).
    __device__ static void dotp(const P &p, const AU &a, float &acc, float &) {
        int isum = 0, bias = 0;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            int sg = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) sg = sdot4(p.q[4 * g + i], a.q[4 * g + i], sg);
            isum += sg * p.sc[g];
            bias += p.sc[g] * a.bs[g];
        }
        acc = fmaf((float)(isum - 32 * bias), p.d * a.d, acc);
    }
    __device__ static void dot(const W &w, uint32_t u, const AU &a, float &acc, float &corr) {
        dotp(prep(w, u), a, acc, corr);
    }
};

// The 32-weight formats, one block per unit, against A8: Q8_0 and IQ4_NL (vecdot.zig:235-250,
// 369-384) signed; Q4_0 / Q5_0 with their zero point subtracted per weight (so the block sum is
// dotQ4_0's dpu - 8*s, dotQ5_0's - 16*s); Q4_1 / Q5_1 unsigned plus m * (d_a * s), with s the
// block's activation sum (dotQ4_1 / dotQ5_1, 311-367).
template <int T> struct MvLegacy {
    static constexpr bool kq = false;
    static constexpr uint32_t QB = (T == HKHIP_Q8_0) ? 32 : 16; // quant-plane bytes per block
    __device__ static uint32_t units(uint32_t K) { return K / 32; }
    __device__ static uint32_t lds_chunk(uint32_t c) { return swz<1>(c); }
    __device__ static uint32_t bs_index(uint32_t g) { return g; }
    struct W {
        uint4 x0, x1;
        uint32_t d, m, qh;
    };
    struct AU {
        uint32_t q[8];
        float d;
    };
    __device__ static RowRef row(const uint8_t *w, const uint16_t *ws, uint32_t r, uint32_t K) {
        const uint32_t nbr = K / 32;
        const SideGeom G = side_geom(T, nbr);
        const uint8_t *side = reinterpret_cast<const uint8_t *>(ws) + uint64_t(r) * G.stride;
        return RowRef{w + uint64_t(r) * nbr * QB, reinterpret_cast<const uint16_t *>(side),
                      reinterpret_cast<const uint16_t *>(side + G.m_off), reinterpret_cast<const uint32_t *>(side + G.qh_off)};
    }
    __device__ static W load(const RowRef &R, uint32_t u) {
        W w;
        w.x0 = ldw(R.w + u * QB);
        if constexpr (T == HKHIP_Q8_0) w.x1 = ldw(R.w + u * QB + 16);
        w.d = R.ws[u];
        if constexpr (has_m(T)) w.m = R.wm[u];
        if constexpr (has_qh(T)) w.qh = R.wh[u];
        return w;
    }
    __device__ static AU act(const ActL &A, uint32_t t, uint32_t u) {
        const uint32_t base = t * (A.K / 16);
        const uint4 v0 = ldw(A.qs + 16 * (base + swz<1>(2 * u)));
        const uint4 v1 = ldw(A.qs + 16 * (base + swz<1>(2 * u + 1)));
        AU a;
        a.q[0] = v0.x; a.q[1] = v0.y; a.q[2] = v0.z; a.q[3] = v0.w;
        a.q[4] = v1.x; a.q[5] = v1.y; a.q[6] = v1.z; a.q[7] = v1.w;
        a.d = A.d[t * (A.K / 32) + u];
        return a;
    }
    // Weight-side work of a unit: its 32 int8 weights (codebook lookups for IQ4_NL, zero point
    // and fifth bits for Q4_0..Q5_1), scale and offset.
    struct P {
        uint32_t q[8];
        float d, m;
    };
    __device__ static P prep(const W &w, uint32_t) {
        P p;
        if constexpr (T == HKHIP_Q8_0) {
            p.q[0] = w.x0.x; p.q[1] = w.x0.y; p.q[2] = w.x0.z; p.q[3] = w.x0.w;
            p.q[4] = w.x1.x; p.q[5] = w.x1.y; p.q[6] = w.x1.z; p.q[7] = w.x1.w;
        } else {
            const uint32_t n4[4] = {w.x0.x, w.x0.y, w.x0.z, w.x0.w};
            const uint32_t qh = has_qh(T) ? w.qh : 0u;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p.q[i] = low_bit_word<T>(n4[i], qh, 0, i);
                p.q[4 + i] = low_bit_word<T>(n4[i], qh, 1, i);
            }
        }
        p.d = f16_bits_to_f32(w.d);
        p.m = has_m(T) ? f16_bits_to_f32(w.m) : 0.0f;
        return p;
    }
    __device__ static void dotp(const P &p, const AU &a, float &acc, float &) {
        int s = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) s = sdot4(p.q[i], a.q[i], s);
        acc = fmaf((float)s, p.d * a.d, acc);
        if constexpr (has_m(T)) {
            int as = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) as = sdot4(0x01010101, a.q[i], as);
            acc = fmaf(p.m, a.d * (float)as, acc);
        }
    }
    __device__ static void dot(const W &w, uint32_t u, const AU &a, float &acc, float &corr) {
        dotp(prep(w, u), a, acc, corr);
    }
};
template <> struct MvFmt<HKHIP_Q8_0> : MvLegacy<HKHIP_Q8_0> {};
template <> struct MvFmt<HKHIP_IQ4_NL> : MvLegacy<HKHIP_IQ4_NL> {};
template <> struct MvFmt<HKHIP_Q4_0> : MvLegacy<HKHIP_Q4_0> {};
template <> struct MvFmt<HKHIP_Q4_1> : MvLegacy<HKHIP_Q4_1> {};
template <> struct MvFmt<HKHIP_Q5_0> : MvLegacy<HKHIP_Q5_0> {};
template <> struct MvFmt<HKHIP_Q5_1> : MvLegacy<HKHIP_Q5_1> {};

// ---------------------------------------------------------------------------------------------
// Shared pieces of the kernels
// ---------------------------------------------------------------------------------------------


// Sum over each aligned group of 2^lg lanes; every lane of the group gets the sum.
__device__ __forceinline__ float group_sum(float v, uint32_t lg) {
    if (lg >= 1) v += dpp_f<DPP_XOR1>(v);
    if (lg >= 2) v += dpp_f<DPP_XOR2>(v);
    if (lg >= 3) v += dpp_f<DPP_HALF_MIRROR>(v);
    if (lg >= 4) v += dpp_f<DPP_MIRROR>(v);
    if (lg == 5) v += __shfl_xor(v, 16);
    if (lg == 6) v = (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
    return v;
}

// Quantizes (or copies) the NT-token input into LDS. All NW waves take part; ends with a barrier.
template <typename F, int NT, int NW>
__device__ __forceinline__ void stage_acts(const MvArgs &a, int8_t *sqs, int16_t *sbs, float *sd) {
    constexpr bool kq = F::kq;
    constexpr uint32_t NTH = NW * 64;
    const uint32_t K = a.K, kc = K / 16;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (a.x) {
        if constexpr (kq) {
            const uint32_t kb = K / 256, nblk = NT * kb;
            // Every load of the first blocks first, then the reductions.
            constexpr int PB = 2;
            float4 xv[PB];
#pragma unroll
            for (int j = 0; j < PB; j++) {
                const uint32_t b = wave + NW * j;
                if (b < nblk) xv[j] = reinterpret_cast<const float4 *>(a.x + uint64_t(b) * 256)[lane];
            }
            auto put = [&](uint32_t b, const Q8KQ &qr) {
                const uint32_t t = NT == 1 ? 0 : b / kb, sb = b - t * kb;
                const uint32_t c = 16 * sb + (lane >> 2);
                *reinterpret_cast<uint32_t *>(sqs + 16 * (t * kc + F::lds_chunk(c)) + 4 * (lane & 3)) = qr.packed;
                if ((lane & 3) == 0) sbs[t * kc + F::bs_index(16 * sb + lane / 4)] = (int16_t)qr.bsum;
                if (lane == 0) sd[b] = qr.d;
            };
#pragma unroll
            for (int j = 0; j < PB; j++) {
                const uint32_t b = wave + NW * j;
                if (b < nblk) put(b, quant_q8k_wave(xv[j], lane));
            }
            for (uint32_t b = wave + NW * PB; b < nblk; b += NW)
                put(b, quant_q8k_wave(reinterpret_cast<const float4 *>(a.x + uint64_t(b) * 256)[lane], lane));
        } else {
            const uint32_t ka = K / 32, nblk = NT * ka, hw = tid >> 5, hl = tid & 31;
            // Both half-waves run every iteration (the quantizer needs the whole wave).
            const uint32_t nb2 = (nblk + 2 * NW - 1) / (2 * NW) * (2 * NW);
            constexpr int PB = 2;
            float xs[PB];
#pragma unroll
            for (int j = 0; j < PB; j++) {
                const uint32_t b = hw + 2 * NW * j;
                xs[j] = b < nblk ? a.x[uint64_t(b) * 32 + hl] : 0.0f;
            }
            auto put = [&](uint32_t b, const A8Q &qr) {
                const uint32_t t = NT == 1 ? 0 : b / ka, blk = b - t * ka;
                sqs[16 * (t * kc + F::lds_chunk(2 * blk + (hl >> 4))) + (hl & 15)] = (int8_t)qr.q;
                if (hl == 0) sd[b] = qr.d;
            };
#pragma unroll
            for (int j = 0; j < PB; j++) {
                if (2 * NW * j < nb2) {
                    const A8Q qr = quant_a8_halfwave(xs[j]);
                    const uint32_t b = hw + 2 * NW * j;
                    if (b < nblk) put(b, qr);
                }
            }
            for (uint32_t b0 = 2 * NW * PB; b0 < nb2; b0 += 2 * NW) {
                const uint32_t b = b0 + hw;
                const A8Q qr = quant_a8_halfwave(b < nblk ? a.x[uint64_t(b) * 32 + hl] : 0.0f);
                if (b < nblk) put(b, qr);
            }
        }
    } else {
        for (uint32_t i = tid; i < NT * kc; i += NTH) {
            const uint32_t t = NT == 1 ? 0 : i / kc, c = i - t * kc;
            reinterpret_cast<uint4 *>(sqs)[t * kc + F::lds_chunk(c)] = reinterpret_cast<const uint4 *>(a.gqs)[i];
        }
        const uint32_t nd = NT * (K / (kq ? 256 : 32));
        for (uint32_t i = tid; i < nd; i += NTH) sd[i] = a.gd[i];
        if constexpr (kq) {
            for (uint32_t i = tid; i < NT * kc; i += NTH) {
                const uint32_t t = NT == 1 ? 0 : i / kc, g = i - t * kc;
                sbs[t * kc + F::bs_index(g)] = a.gbs[i];
            }
        }
    }
    __syncthreads();
}

#define MV_SEL(f) (p == 0 ? a.p[0].f : p == 1 ? a.p[1].f : p == 2 ? a.p[2].f : a.p[3].f)

// The row group g of a wave: its part (the same for every lane), local row and row pointers.
template <typename F>
__device__ __forceinline__ RowRef mv_locate(const MvArgs &a, uint32_t g, uint32_t sub, uint32_t rpw, uint32_t &p,
                                            uint32_t &r, bool &active) {
    p = 0;
#pragma unroll
    for (int i = 1; i < MV_PARTS; i++)
        if (i < int(a.nparts) && g >= a.p[i].gstart) p = i;
    r = (g - MV_SEL(gstart)) * rpw + sub;
    active = r < MV_SEL(rows);
    return F::row(MV_SEL(w), MV_SEL(ws), active ? r : 0, a.K);
}

template <int NT>
__device__ __forceinline__ void mv_store(const MvArgs &a, uint32_t p, uint32_t r, const float *acc) {
    float *y = MV_SEL(y);
    const float *bias = MV_SEL(bias);
    const uint32_t rows = MV_SEL(rows);
    const float b = bias ? bias[r] : 0.0f;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        float *dst = y + uint64_t(t) * rows + r;
        if (a.mode == HKHIP_ACCUMULATE)
            *dst += acc[t] + b;
        else
            *dst = acc[t] + b;
    }
}

// ---------------------------------------------------------------------------------------------
// General kernel: NT tokens, rows of any length (steps of UNR units per lane), activations from
// LDS.
// ---------------------------------------------------------------------------------------------

template <int T, int NT, int NW, int UNR>
__global__ __launch_bounds__(NW * 64) void mmvq_kernel(MvArgs a) {
    using F = MvFmt<T>;
    using W = typename F::W;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr bool kq = F::kq;
    const uint32_t K = a.K;
    int8_t *sqs = reinterpret_cast<int8_t *>(smem);
    int16_t *sbs = reinterpret_cast<int16_t *>(smem + NT * K);
    float *sd = reinterpret_cast<float *>(smem + NT * K + (kq ? NT * K / 8 : 0));
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t lg = a.lpr_log2, lpr = 1u << lg, rpw = 64u >> lg;
    const uint32_t sub = lane >> lg, ul = lane & (lpr - 1);
    const uint32_t U = F::units(K);
    const uint32_t step_units = UNR * lpr;
    const uint32_t nch = (U + step_units - 1) / step_units; // steps per row
    const uint32_t nwaves = gridDim.x * NW, wid = blockIdx.x * NW + wave;
    const uint32_t g0 = uint32_t(uint64_t(a.ngroups) * wid / nwaves);
    const uint32_t g1 = uint32_t(uint64_t(a.ngroups) * (wid + 1) / nwaves);

    stage_acts<F, NT, NW>(a, sqs, sbs, sd);
    const ActL act{sqs, sbs, sd, K};

    float acc[NT], corr[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = corr[t] = 0.0f;
    W wa[UNR], wb[UNR];
    auto load = [&](W *w, uint32_t g, uint32_t ch) {
        uint32_t p, r;
        bool active;
        const RowRef R = mv_locate<F>(a, g, sub, rpw, p, r, active);
        const uint32_t base = ul + ch * step_units;
#pragma unroll
        for (int c = 0; c < UNR; c++) {
            const uint32_t u = base + c * lpr;
            if (active && u < U) w[c] = F::load(R, u);
        }
    };
    auto compute = [&](const W *w, uint32_t g, uint32_t ch) {
        uint32_t p, r;
        bool active;
        (void)mv_locate<F>(a, g, sub, rpw, p, r, active);
        const uint32_t base = ul + ch * step_units;
        if (active) {
#pragma unroll
            for (int c = 0; c < UNR; c++) {
                const uint32_t u = base + c * lpr;
                if (u < U) {
#pragma unroll
                    for (int t = 0; t < NT; t++) F::dot(w[c], u, F::act(act, t, u), acc[t], corr[t]);
                }
            }
        }
        if (ch + 1 < nch) return;
        float v[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            v[t] = group_sum(acc[t] - corr[t], lg);
            acc[t] = corr[t] = 0.0f;
        }
        if (a.mode == HKHIP_SILU_MUL) {
            // Row r's lanes are sub-group `sub`; the up row of an even r is the next sub-group
            // (the launch keeps at least two rows per wave in this mode).
            float up[NT];
#pragma unroll
            for (int t = 0; t < NT; t++) up[t] = __shfl_down(v[t], lpr);
            if (active && ul == 0 && (r & 1) == 0) {
                float *y = MV_SEL(y);
                const uint32_t rows = MV_SEL(rows);
#pragma unroll
                for (int t = 0; t < NT; t++) y[uint64_t(t) * (rows / 2) + r / 2] = silu_mul(v[t], up[t]);
            }
        } else if (active && ul == 0) {
            mv_store<NT>(a, p, r, v);
        }
    };
    // Steps in order (g, ch); the next step's weights load while this one computes.
    uint32_t g = g0, ch = 0;
    if (g < g1) load(wa, g, ch);
    while (g < g1) {
        uint32_t gn = g, cn = ch + 1;
        if (cn == nch) {
            gn++;
            cn = 0;
        }
        if (gn < g1) load(wb, gn, cn);
        compute(wa, g, ch);
        if (gn >= g1) break;
        uint32_t g2 = gn, c2 = cn + 1;
        if (c2 == nch) {
            g2++;
            c2 = 0;
        }
        if (g2 < g1) load(wa, g2, c2);
        compute(wb, gn, cn);
        g = g2;
        ch = c2;
    }
}

// ---------------------------------------------------------------------------------------------
// Register kernel: lane l of every wave owns units l, l+64, ... (C of them) of every row, and
// keeps their activations for all NT tokens in registers. A wave streams whole rows, R rows per
// step (one token: step s of wave group g takes the step-sized row chunk s * groups + g, so that
// each step's loads across the grid cover one contiguous span of the matrix, which measured
// faster than a contiguous row range per wave; several tokens: a contiguous range, as their
// kernels have no registers to spare), so row addresses are wave-uniform (scalar) and each activation
// register is reused for every row. There is no LDS and no barrier: the first step's weight
// loads are issued before the activations are read, and an f32 input is quantized by the lanes
// themselves (a Q8K super-block is four consecutive units, i.e. four neighbouring lanes).
// ---------------------------------------------------------------------------------------------

// Unit u of token t from quantized activations in the engine's layout (global memory or LDS):
// qs [n][K] int8, bs [n][K/16] int16 (Q8K), d [n][K/256] (Q8K) or [n][K/32] (A8) f32.
template <typename F>
__device__ __forceinline__ typename F::AU load_unit(const int8_t *gqs, const int16_t *gbs, const float *gd, uint32_t K,
                                                    uint32_t t, uint32_t u) {
    typename F::AU au;
    if constexpr (F::kq) {
        const int8_t *qs = gqs + uint64_t(t) * K;
        uint32_t q[16];
        int bs[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t off = F::chunk_off(u, j);
            const uint4 v = ldw(qs + off);
            q[4 * j] = v.x; q[4 * j + 1] = v.y; q[4 * j + 2] = v.z; q[4 * j + 3] = v.w;
            bs[j] = gbs[uint64_t(t) * (K / 16) + off / 16];
        }
        au = F::make(q, bs, gd[t * (K / 256) + (u >> 2)]);
    } else {
        const int8_t *qs = gqs + uint64_t(t) * K + 32 * u;
        const uint4 v0 = ldw(qs), v1 = ldw(qs + 16);
        au.q[0] = v0.x; au.q[1] = v0.y; au.q[2] = v0.z; au.q[3] = v0.w;
        au.q[4] = v1.x; au.q[5] = v1.y; au.q[6] = v1.z; au.q[7] = v1.w;
        au.d = gd[t * (K / 32) + u];
    }
    return au;
}

// Bytes of LDS the register kernel uses to stage an f32 input of nt tokens.
__host__ __device__ inline uint32_t mvr_lds_bytes(int nt, uint32_t K, bool kq) {
    return nt * K + (kq ? nt * K / 8 + nt * (K / 256) * 4 : nt * (K / 32) * 4);
}
// The fused norm's per-lane sums follow the staging area and the K-slice partials (`extra`).
__host__ __device__ inline uint32_t mvr_norm_offset(uint32_t nt, uint32_t K, bool kq, uint32_t extra) {
    return ((mvr_lds_bytes(int(nt), K, kq) + 15) & ~15u) + extra;
}

// Quantizes 1024 consecutive inputs per wave (lane l holds values 16l..16l+15 of the chunk) with
// the qact arithmetic and writes them to the LDS staging area in the engine's activation layout.
// Q8K: a block of 256 is one row of 16 lanes, so every reduction stays inside a DPP row and a
// wave quantizes four blocks at once. A8: a block of 32 is two lanes. `valid` is false for lanes
// past the input (whole blocks). All 64 lanes must execute this.
template <typename F>
__device__ __forceinline__ void mvr_stage_chunk(const float4 *xv, uint32_t c, bool valid, int8_t *sqs,
                                                int16_t *sbs, float *sd) {
    const uint32_t lane = __lane_id();
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[4 * i] = xv[i].x; v[4 * i + 1] = xv[i].y; v[4 * i + 2] = xv[i].z; v[4 * i + 3] = xv[i].w;
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(v[i]));
    const uint32_t e = 1024 * c + 16 * lane; // first input of this lane
    uint32_t pk[4];
    if constexpr (F::kq) {
        const float amax = row_max(m);
        // Signed value of the first element with |x| == amax (lowest index wins, as the
        // reference's strict '>' scan does): this lane's first hit, then the row's lowest lane.
        float first = 0.0f;
        bool hit = false;
#pragma unroll
        for (int i = 15; i >= 0; i--) {
            if (fabsf(v[i]) == amax) {
                first = v[i];
                hit = true;
            }
        }
        const uint64_t mask = __ballot(hit);
        const uint32_t rbits = uint32_t(mask >> (lane & 48)) & 0xFFFFu;
        const float mx = __shfl(first, int((lane & 48) + (rbits ? __builtin_ctz(rbits) : 0)));
        const bool zero = amax == 0.0f || rbits == 0;
        const float iscale = zero ? 0.0f : __fdiv_rn(-127.0f, mx);
        int bsum = 0;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            uint32_t p = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int t = (int)roundf(iscale * v[4 * w + b]);
                p |= uint32_t(uint8_t(t < 127 ? t : 127)) << (8 * b);
            }
            pk[w] = p;
            bsum = sdot4(p, 0x01010101u, bsum);
        }
        if (valid) {
            *reinterpret_cast<uint4 *>(sqs + e) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            sbs[e / 16] = (int16_t)bsum;
            if ((lane & 15) == 0) sd[e / 256] = zero ? 0.0f : __fdiv_rn(1.0f, iscale);
        }
    } else {
        const float amax = fmaxf(m, dpp_f<DPP_XOR1>(m));
        const float d = __fdiv_rn(amax, 127.0f);
        const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            uint32_t p = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) p |= uint32_t(uint8_t((int)roundf(v[4 * w + b] * id))) << (8 * b);
            pk[w] = p;
        }
        if (valid) {
            *reinterpret_cast<uint4 *>(sqs + e) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            if ((lane & 1) == 0) sd[e / 32] = d;
        }
    }
}

// KS > 1 splits each row's units over KS waves of a workgroup (for rows whose activations would
// not fit one wave's registers): wave w is slice w % KS of row group w / KS; the slices' partial
// results meet in LDS at the end.
// LG < 6 packs short rows: a row takes 2^LG lanes (one unit each, C = 1), so a wave covers
// 64 >> LG rows per row slot and step and its row addresses are per lane.
template <int T, int NT, int C, int R, int NW, int KS, int LG = 6, bool NORM = true>
__global__ __launch_bounds__(NW * 64) void mmvr_kernel(MvArgs a) {
    using F = MvFmt<T>;
    using W = typename F::W;
    using AU = typename F::AU;
    static_assert(NW % KS == 0, "slices per workgroup");
    static_assert(LG == 6 || (C == 1 && KS == 1), "packed rows: one unit per lane, one slice");
    constexpr int NRG = NW / KS; // row groups per workgroup
    constexpr uint32_t LPR = 1u << LG, G = 64u >> LG, RS = R * G; // lanes per row, rows per slot, rows per step
    const uint32_t K = a.K;
    const uint32_t lane = __lane_id();
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t rg = wave / KS, ks = wave % KS;
    const uint32_t U = F::units(K);
    const uint32_t u0 = ks * 64 * C; // first unit of this wave's slice
    const uint32_t ul = LG == 6 ? lane : (lane & (LPR - 1)), sub = LG == 6 ? 0u : lane >> LG; // unit lane, row in slot
    const uint32_t ngroups = gridDim.x * NRG, gid = blockIdx.x * NRG + rg;
    const uint32_t total = a.ngroups; // rows of all parts
    // Mode HKHIP_SILU_MUL splits the rows in gate/up pairs, so that a pair stays in one wave.
    const uint32_t pr = a.mode == HKHIP_SILU_MUL ? 2u : 1u;
    // Interleaved: step st of this group covers rows (st * ngroups + gid) * RS .. + RS - 1 (clamped
    // to the last row); contiguous: rows r0 .. r1 - 1, RS per step.
    // One token only (the multi-token kernels are at the register limit), and not where a step's
    // rows would split a gate/up pair.
    const bool il = NT == 1 && a.interleave != 0 && (a.mode != HKHIP_SILU_MUL || RS % 2 == 0);
    const uint32_t nch = (total + RS - 1) / RS;
    const uint32_t r0 = il ? 0u : pr * uint32_t(uint64_t(total / pr) * gid / ngroups);
    const uint32_t r1 = il ? total : pr * uint32_t(uint64_t(total / pr) * (gid + 1) / ngroups);
    // A wave without rows still helps stage the input (and reaches the barrier).
    const uint32_t rlast = r0 < r1 ? r1 - 1 : 0;
    auto base = [&](uint32_t st) -> uint32_t { return il ? (st * ngroups + gid) * RS : r0 + st * RS; };
    // Row whose result lane j keeps (lane j = step j / RS, row j % RS of the step).
    auto row_of = [&](uint32_t j) -> uint32_t { return il ? base(j / RS) + j % RS : r0 + j; };

    // Row r of the concatenated parts: its part. Fields are copied member by member so the
    // argument block is never indexed dynamically (which would move it to scratch).
    auto locate = [&](uint32_t r) -> MvPart {
        MvPart q = a.p[0];
#pragma unroll
        for (int i = 1; i < MV_PARTS; i++) {
            if (i < int(a.nparts) && r >= a.p[i].gstart) {
                q.w = a.p[i].w;
                q.ws = a.p[i].ws;
                q.y = a.p[i].y;
                q.bias = a.p[i].bias;
                q.rows = a.p[i].rows;
                q.gstart = a.p[i].gstart;
            }
        }
        return q;
    };
    // Every step issues the same loads, with rows past the range and units past the row clamped
    // to valid ones, and no other global load happens until the final stores: the compiler can
    // then wait for exactly the older step while the newer one stays in flight (the memory
    // counter is in order, so any later load that is waited on would drain the prefetch too).
    W wa[R][C], wb[R][C];
    auto load = [&](W (*w)[C], uint32_t rb) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uint32_t r = rb + i * G + sub < r1 ? rb + i * G + sub : rlast;
            const MvPart q = locate(r);
            const RowRef RR = F::row(q.w, q.ws, r - q.gstart, K);
#pragma unroll
            for (int c = 0; c < C; c++) {
                const uint32_t u = u0 + ul + LPR * c;
                w[i][c] = F::load(RR, u < U ? u : U - 1);
            }
        }
    };
    // Activations. An f32 input is quantized once per workgroup into LDS: its first blocks are
    // loaded before any weight, so quantizing them waits only for them (the memory counter is
    // in order), and the weights of the first two steps stream in meanwhile. A quantized input
    // is read by each lane directly, also ahead of the weights.
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t ntok = NT == 1 ? 1u : a.ntok;
    const uint32_t nflat = ntok * K;
    // Chunks of 1024 inputs per wave: at most NT*K/1024/NW = (4 or 2)*NT*C/NW. Up to 4 are
    // loaded up front (clamped, always issued).
    constexpr int PB = mvr_pb(F::kq, NT, C, NW);
    const uint32_t nchunk = (nflat + 1023) / 1024;
    float4 xv[PB][4];
    AU au[NT][C];
    auto xload = [&](uint32_t cidx, float4 *dst) {
        const uint32_t e = 1024 * (cidx < nchunk ? cidx : nchunk - 1) + 16 * lane;
        const float4 *src = reinterpret_cast<const float4 *>(a.x + (e < nflat ? e : nflat - 16));
#pragma unroll
        for (int i = 0; i < 4; i++) dst[i] = src[i];
    };
    // The fused norm's weights of those chunks too, before any weight row: loaded after them, the
    // staging would wait for the first step's rows (the memory counter is in order).
    float4 nv[NORM ? PB : 1][4];
    if (a.x) {
#pragma unroll
        for (int j = 0; j < PB; j++) xload(wave + NW * j, xv[j]);
        if (NORM && a.norm) {
#pragma unroll
            for (int j = 0; j < PB; j++) {
                const uint32_t cidx = wave + NW * j, e = 1024 * (cidx < nchunk ? cidx : nchunk - 1) + 16 * lane;
                const float4 *wv = reinterpret_cast<const float4 *>(a.norm + (e < nflat ? e % K : 0));
#pragma unroll
                for (int i = 0; i < 4; i++) nv[NORM ? j : 0][i] = wv[i];
            }
        }
    } else {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (NT > 1 && uint32_t(t) >= a.ntok) break;
#pragma unroll
            for (int c = 0; c < C; c++) {
                const uint32_t u = u0 + ul + LPR * c;
                au[t][c] = load_unit<F>(a.gqs, a.gbs, a.gd, K, t, u < U ? u : U - 1);
            }
        }
    }
    const uint32_t ns = il ? (gid < nch ? (nch - gid + ngroups - 1) / ngroups : 0u)
                           : (r1 - r0 + RS - 1) / RS; // steps of this wave
    const uint32_t nres = il ? (ns * RS) : r1 - r0;  // lanes holding a result (rows past the end skipped)
    load(wa, base(0));
    if (a.x) {
        int8_t *sqs = reinterpret_cast<int8_t *>(smem);
        int16_t *sbs = reinterpret_cast<int16_t *>(smem + nflat);
        float *sd = reinterpret_cast<float *>(smem + nflat + (F::kq ? nflat / 8 : 0));
        // Fused RMS norm: per-lane sums of squares of 16 inputs to LDS (the first chunks from the
        // registers, any further ones loaded once more), then every wave adds a token's sums in
        // one fixed order, so all workgroups get the same factor.
        // The tokens' factors go to LDS (after the partial sums), not registers: NT of them live
        // through the staging pushed the 8-token kernels into spills.
        float *sinv = reinterpret_cast<float *>(smem + mvr_norm_offset(ntok, K, F::kq, KS > 1 ? NW * 64 * NT * 4 : 0)) + nflat / 16;
        auto norm_chunk = [&](float4 *v, uint32_t e, const float4 *w) { // w: the weights, or null (loaded here)
            const float inv = sinv[e < nflat ? e / K : 0];
            const float4 *wv = reinterpret_cast<const float4 *>(a.norm + (e < nflat ? e % K : 0));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 w4 = w ? w[i] : wv[i];
                v[i].x = (v[i].x * inv) * w4.x;
                v[i].y = (v[i].y * inv) * w4.y;
                v[i].z = (v[i].z * inv) * w4.z;
                v[i].w = (v[i].w * inv) * w4.w;
            }
        };
        if (NORM && a.norm) {
            float *parts = reinterpret_cast<float *>(smem + mvr_norm_offset(ntok, K, F::kq, KS > 1 ? NW * 64 * NT * 4 : 0));
            auto sumsq = [&](const float4 *v, uint32_t e) {
                float ss = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    ss = fmaf(v[i].x, v[i].x, ss);
                    ss = fmaf(v[i].y, v[i].y, ss);
                    ss = fmaf(v[i].z, v[i].z, ss);
                    ss = fmaf(v[i].w, v[i].w, ss);
                }
                parts[e / 16] = ss;
            };
#pragma unroll
            for (int j = 0; j < PB; j++) {
                const uint32_t e = 1024 * (wave + NW * j) + 16 * lane;
                if (wave + NW * j < nchunk && e < nflat) sumsq(xv[j], e);
            }
            for (uint32_t c0 = wave + NW * PB; c0 < nchunk; c0 += NW) {
                float4 tmp[4];
                xload(c0, tmp);
                const uint32_t e = 1024 * c0 + 16 * lane;
                if (e < nflat) sumsq(tmp, e);
            }
            __syncthreads();
            // Wave w adds token w's sums (and w + NW, ...), in the same order in every workgroup.
            for (uint32_t t = wave; t < ntok; t += NW) {
                float ss = 0.0f;
                for (uint32_t q = t * (K / 16) + lane; q < (t + 1) * (K / 16); q += 64) ss += parts[q];
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
                if (lane == 0) sinv[t] = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, float(K)) + a.eps));
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < PB; j++) {
                norm_chunk(xv[j], 1024 * (wave + NW * j) + 16 * lane, nv[NORM ? j : 0]);
                asm volatile("" ::: "memory");
            }
        }
#pragma unroll
        for (int j = 0; j < PB; j++) {
            const uint32_t cidx = wave + NW * j;
            if (cidx < nchunk) mvr_stage_chunk<F>(xv[j], cidx, 1024 * cidx + 16 * lane < nflat, sqs, sbs, sd);
        }
        // Rare (more than PB chunks per wave): the rest, PB chunks at a time.
        for (uint32_t c0 = wave + NW * PB; c0 < nchunk; c0 += NW * PB) {
#pragma unroll
            for (int j = 0; j < PB; j++) xload(c0 + NW * j, xv[j]);
            if (NORM && a.norm) {
#pragma unroll
                for (int j = 0; j < PB; j++) norm_chunk(xv[j], 1024 * (c0 + NW * j) + 16 * lane, nullptr);
            }
#pragma unroll
            for (int j = 0; j < PB; j++) {
                const uint32_t cidx = c0 + NW * j;
                if (cidx < nchunk) mvr_stage_chunk<F>(xv[j], cidx, 1024 * cidx + 16 * lane < nflat, sqs, sbs, sd);
            }
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (NT > 1 && uint32_t(t) >= a.ntok) break;
#pragma unroll
            for (int c = 0; c < C; c++) {
                const uint32_t u = u0 + ul + LPR * c;
                au[t][c] = load_unit<F>(sqs, sbs, sd, K, t, u < U ? u : U - 1);
            }
        }
    }
    // The second step is issued only now, so that the barrier does not wait for every wave to get
    // two steps of loads past a busy memory pipeline.
    if (ns > 1) load(wb, base(1));

    // Lane j keeps the result of row row_of(j); the launch gives no wave more than 64 rows, so the
    // results are stored once, at the end, and the loop issues no load but weights.
    float res[NT];
    auto flush = [&](uint32_t n) {
        if (a.mode == HKHIP_SILU_MUL) {
            // Lane 2i holds a gate row, lane 2i + 1 its up row (r0 and the interleaved steps' first
            // rows are even).
            float up[NT];
#pragma unroll
            for (int t = 0; t < NT; t++) up[t] = __shfl_down(res[t], 1);
            if (lane < n && (lane & 1) == 0 && row_of(lane) < total) {
                const MvPart q = locate(row_of(lane));
                const uint32_t o = (row_of(lane) - q.gstart) / 2;
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    if (NT > 1 && uint32_t(t) >= a.ntok) break;
                    q.y[uint64_t(t) * (q.rows / 2) + o] = silu_mul(res[t], up[t]);
                }
            }
            return;
        }
        if (lane < n && row_of(lane) < total) {
            const uint32_t r = row_of(lane);
            MvPart q = a.p[0];
#pragma unroll
            for (int i = 1; i < MV_PARTS; i++) {
                if (i < int(a.nparts) && r >= a.p[i].gstart) {
                    q.y = a.p[i].y;
                    q.bias = a.p[i].bias;
                    q.rows = a.p[i].rows;
                    q.gstart = a.p[i].gstart;
                }
            }
            const uint32_t lr = r - q.gstart;
            const float b = q.bias ? q.bias[lr] : 0.0f;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if (NT > 1 && uint32_t(t) >= a.ntok) break;
                float *y = q.y + uint64_t(t) * q.rows + lr;
                if (a.mode == HKHIP_ACCUMULATE)
                    *y += res[t] + b;
                else
                    *y = res[t] + b;
            }
        }
    };
    auto compute = [&](const W (*w)[C], uint32_t st) {
        const uint32_t rb = base(st);
#pragma unroll
        for (int i = 0; i < R; i++) {
            if (rb + i * G >= r1) break;
            float acc[NT], corr[NT];
#pragma unroll
            for (int t = 0; t < NT; t++) acc[t] = corr[t] = 0.0f;
#pragma unroll
            for (int c = 0; c < C; c++) {
                const uint32_t u = u0 + ul + LPR * c;
                if (u < U) {
                    const typename F::P pw = F::prep(w[i][c], u);
#pragma unroll
                    for (int t = 0; t < NT; t++)
                        if (NT == 1 || uint32_t(t) < a.ntok) F::dotp(pw, au[t][c], acc[t], corr[t]);
                }
            }
            const uint32_t slot = st * RS + i * G; // lane of the slot's first row
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float v = group_sum(acc[t] - corr[t], LG);
                if constexpr (LG == 6) {
                    if (lane == slot) res[t] = v;
                } else {
                    // Row slot + g's sum is in lanes g*LPR..; lane slot + g takes it.
                    const uint32_t g = lane - slot;
                    const float vg = __shfl(v, int((g & (G - 1)) << LG));
                    if (g < G) res[t] = vg;
                }
            }
        }
    };
    // Steady state: every step's loads are valid, so each load is issued unconditionally and the
    // wait before a compute covers exactly the older buffer. The last (up to three) steps are
    // peeled so that nothing is loaded past the range.
    uint32_t s = 0;
    for (; s + 3 < ns; s += 2) {
        compute(wa, s);
        load(wa, base(s + 2));
        compute(wb, s + 1);
        load(wb, base(s + 3));
    }
    auto step = [&](const W (*w)[C], uint32_t st) { compute(w, st); };
    if (s + 2 < ns) {
        step(wa, s);
        load(wa, base(s + 2));
        step(wb, s + 1);
        step(wa, s + 2);
    } else if (s + 1 < ns) {
        step(wa, s);
        step(wb, s + 1);
    } else if (s < ns) {
        step(wa, s);
    }
    if constexpr (KS > 1) {
        // Slices 1.. leave their partials in LDS (after the staging area); slice 0 adds and stores.
        const uint32_t cofs = a.x ? (mvr_lds_bytes(int(NT == 1 ? 1u : a.ntok), K, F::kq) + 15) & ~15u : 0u;
        float *cb = reinterpret_cast<float *>(smem + cofs) + (rg * KS) * 64 * NT;
        if (ks > 0) {
#pragma unroll
            for (int t = 0; t < NT; t++) cb[(ks * 64 + lane) * NT + t] = res[t];
        }
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int k = 1; k < KS; k++)
#pragma unroll
                for (int t = 0; t < NT; t++) res[t] += cb[(k * 64 + lane) * NT + t];
            flush(nres);
        }
    } else {
        flush(nres);
    }
}

#undef MV_SEL

// ---------------------------------------------------------------------------------------------
// Launch
// ---------------------------------------------------------------------------------------------

typedef void (*mv_kernel_t)(MvArgs);

constexpr int MV_NW = 8, MV_UNR = 2;   // general kernel: 8 waves, 2 units per lane per step

template <int T>
mv_kernel_t pick(int nt) {
    switch (nt) {
    case 1: return mmvq_kernel<T, 1, MV_NW, MV_UNR>;
    case 2: return mmvq_kernel<T, 2, MV_NW, MV_UNR>;
    case 3: return mmvq_kernel<T, 3, MV_NW, MV_UNR>;
    case 4: return mmvq_kernel<T, 4, MV_NW, MV_UNR>;
    case 5: return mmvq_kernel<T, 5, MV_NW, MV_UNR>;
    case 6: return mmvq_kernel<T, 6, MV_NW, MV_UNR>;
    case 7: return mmvq_kernel<T, 7, MV_NW, MV_UNR>;
    case 8: return mmvq_kernel<T, 8, MV_NW, MV_UNR>;
    default: return nullptr;
    }
}



// Register kernel variants: NT in {1, 2, 4, 8} (a launch of n tokens uses the smallest NT >= n),
// C = units per lane (rows of at most 64*C units), R = rows per step. The activations of NT*C
// units must fit the register file next to two steps of weights: NT*C <= 8 for Q4_K/Q6_K and
// <= 16 for the 32-weight formats; larger shapes use the LDS kernel.
constexpr int MVR_NWAVES = 8; // waves per workgroup (a budget of 256 registers per lane)
constexpr int MVR_R1 = 2;     // rows per step at one token and C = 1
__host__ __device__ constexpr int mvr_rows(int nt, int c) { return nt == 1 ? (c >= MVR_R1 ? 1 : MVR_R1 / c) : (c >= 2 || nt >= 8 ? 1 : 2); }
// Largest C per (format, NT): the activations of NT*C units must fit the register file next to
// two steps of weights.
__host__ __device__ constexpr int mvr_cmax(int t, int nt) {
    return t == HKHIP_Q4_K || t == HKHIP_IQ4_XS ? (nt == 1 ? 4 : nt == 8 ? 1 : 2)
         : t == HKHIP_Q5_K ? (nt == 1 ? 2 : 1)
         : t == HKHIP_Q6_K ? (nt == 1 ? 4 : nt == 2 ? 2 : 1)
                           : (nt == 1 ? 8 : nt == 8 ? 2 : 4);
}
// Waves per workgroup: MVR_NWAVES (a budget of 256 registers per lane), or 4 (512) for the
// variants that need more.
__host__ __device__ constexpr int mvr_nw(int t, int nt, int c) {
    return ((t == HKHIP_Q6_K || t == HKHIP_Q5_K) && nt * c >= 4) ||
                   ((t == HKHIP_Q4_K || t == HKHIP_IQ4_XS) && nt * c >= 8 && nt < 8) ||
                   (legacy32(t) && c >= 4 && nt * c >= 8)
               ? 4
               : MVR_NWAVES;
}

// NORM: the variant with the fused RMS norm of the input (the 8-token kernels also come without
// it: its staging code alone pushed them past the register file, 21 -> 28 us for the 8B gate/up).
template <int T, int NT, int C, int KS, bool NORM>
mv_kernel_t mvr_if_fits() {
    if constexpr (C <= mvr_cmax(T, NT) && KS <= mvr_nw(T, NT, C))
        return mmvr_kernel<T, NT, C, mvr_rows(NT, C), mvr_nw(T, NT, C), KS, 6, NORM>;
    else
        return nullptr;
}

// Units per lane c and slices ks: one slice for c <= cmax; beyond that, the largest c (cmax) in
// 2, 4 or 8 slices.
template <int T, int NT, bool NORM>
mv_kernel_t mvr_pick_c(int c, int ks) {
    constexpr int CM = mvr_cmax(T, NT);
    if (ks == 1) {
        switch (c) {
        case 1: return mvr_if_fits<T, NT, 1, 1, NORM>();
        case 2: return mvr_if_fits<T, NT, 2, 1, NORM>();
        case 4: return mvr_if_fits<T, NT, 4, 1, NORM>();
        case 8: return mvr_if_fits<T, NT, 8, 1, NORM>();
        default: return nullptr;
        }
    }
    if (c != CM) return nullptr;
    switch (ks) {
    case 2: return mvr_if_fits<T, NT, CM, 2, NORM>();
    case 4: return mvr_if_fits<T, NT, CM, 4, NORM>();
    case 8: return mvr_if_fits<T, NT, CM, 8, NORM>();
    default: return nullptr;
    }
}

// One token, rows of at most 64 units (C = 1): 2^lg lanes per row (lg 4: 4 rows per row slot, 5: 2,
// 6: 1), nw waves per workgroup; nw 8 with two row slots per step is the streaming configuration,
// nw 1-4 with one slot the short-launch one.
template <int T, int LG>
mv_kernel_t mvs_pick_nw(int nw) {
    switch (nw) {
    case 1: return mmvr_kernel<T, 1, 1, 1, 1, 1, LG>;
    case 2: return mmvr_kernel<T, 1, 1, 1, 2, 1, LG>;
    case 4: return mmvr_kernel<T, 1, 1, 1, 4, 1, LG>;
    case 8: return mmvr_kernel<T, 1, 1, 2, 8, 1, LG>;
    default: return nullptr;
    }
}
template <int T>
mv_kernel_t mvs_pick(int lg, int nw) {
    switch (lg) {
    case 4: return mvs_pick_nw<T, 4>(nw);
    case 5: return mvs_pick_nw<T, 5>(nw);
    case 6: return mvs_pick_nw<T, 6>(nw);
    default: return nullptr;
    }
}

template <int T>
mv_kernel_t mvr_pick(int nt, int c, int ks, bool norm) {
    switch (nt) {
    case 1: return mvr_pick_c<T, 1, true>(c, ks);
    case 2: return mvr_pick_c<T, 2, true>(c, ks);
    case 4: return mvr_pick_c<T, 4, true>(c, ks);
    case 8: return norm ? mvr_pick_c<T, 8, true>(c, ks) : mvr_pick_c<T, 8, false>(c, ks);
    default: return nullptr;
    }
}

// Each format's kernels are instantiated in a translation unit of their own (mmvq_<format>.hip),
// so the library builds in parallel; everything else only refers to them.
#ifndef MMVQ_INSTANTIATE
extern template mv_kernel_t pick<HKHIP_Q4_K>(int);
extern template mv_kernel_t mvr_pick<HKHIP_Q4_K>(int, int, int, bool);
extern template mv_kernel_t mvs_pick<HKHIP_Q4_K>(int, int);
extern template mv_kernel_t pick<HKHIP_Q6_K>(int);
extern template mv_kernel_t mvr_pick<HKHIP_Q6_K>(int, int, int, bool);
extern template mv_kernel_t mvs_pick<HKHIP_Q6_K>(int, int);
extern template mv_kernel_t pick<HKHIP_Q5_K>(int);
extern template mv_kernel_t mvr_pick<HKHIP_Q5_K>(int, int, int, bool);
extern template mv_kernel_t mvs_pick<HKHIP_Q5_K>(int, int);
extern template mv_kernel_t pick<HKHIP_IQ4_XS>(int);
extern template mv_kernel_t mvr_pick<HKHIP_IQ4_XS>(int, int, int, bool);
extern template mv_kernel_t mvs_pick<HKHIP_IQ4_XS>(int, int);
extern template mv_kernel_t pick<HKHIP_Q8_0>(int);
extern template mv_kernel_t mvr_pick<HKHIP_Q8_0>(int, int, int, bool);
extern template mv_kernel_t mvs_pick<HKHIP_Q8_0>(int, int);
extern template mv_kernel_t pick<HKHIP_IQ4_NL>(int);
extern template mv_kernel_t mvr_pick<HKHIP_IQ4_NL>(int, int, int, bool);
extern template mv_kernel_t mvs_pick<HKHIP_IQ4_NL>(int, int);
extern template mv_kernel_t pick<HKHIP_Q4_0>(int);
extern template mv_kernel_t mvr_pick<HKHIP_Q4_0>(int, int, int, bool);
extern template mv_kernel_t mvs_pick<HKHIP_Q4_0>(int, int);
extern template mv_kernel_t pick<HKHIP_Q4_1>(int);
extern template mv_kernel_t mvr_pick<HKHIP_Q4_1>(int, int, int, bool);
extern template mv_kernel_t mvs_pick<HKHIP_Q4_1>(int, int);
extern template mv_kernel_t pick<HKHIP_Q5_0>(int);
extern template mv_kernel_t mvr_pick<HKHIP_Q5_0>(int, int, int, bool);
extern template mv_kernel_t mvs_pick<HKHIP_Q5_0>(int, int);
extern template mv_kernel_t pick<HKHIP_Q5_1>(int);
extern template mv_kernel_t mvr_pick<HKHIP_Q5_1>(int, int, int, bool);
extern template mv_kernel_t mvs_pick<HKHIP_Q5_1>(int, int);
#endif

} // namespace hkhip
