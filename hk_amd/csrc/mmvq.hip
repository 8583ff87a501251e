// Decode matvec (mmvq): y[t][r] = dot(W[r], x[t]) for 1..8 tokens, straight from the quantized
// weights. Integer parts follow src/quant/vecdot.zig exactly (dotQ8_0 235-250, dotIQ4NL 369-384,
// k4Block/dotQ4K 482-522, dotQ6K 533-570); only the order of the f32 scale accumulation differs.
//
// One launch computes up to four matrices that read the same input (q/k/v, gate/up), the way
// matmul.runParts fuses them on the CPU (src/engine/matmul.zig:96-144). Each workgroup stages
// the quantized activations in LDS: either it quantizes the f32 input itself with the qact
// arithmetic (quant.hpp; every workgroup produces the same bytes), or it copies an input already
// quantized by hkhip_qact. A wave issues the weight loads of its first rows before that staging,
// so the activation work hides under the HBM latency instead of adding to it.
//
// Mapping: a row is owned by `lpr` lanes of one wave, chosen so each lane holds up to four work
// units of the row (a 4096-wide Q4_K row: 16 lanes x 4 units, four rows per wave). A unit is the
// slice of a row a lane handles, chosen so every lane issues 16-byte loads:
//   Q4_K   a quarter super-block: 32 B of nibbles (two sub-blocks of 32) + the 16-B header
//   Q6_K   a quarter super-block: 16 B of each of ql-low, ql-high, qh (64 weights, 4 groups)
//   Q8_0   one block: 32 B of int8
//   IQ4_NL one block: 16 B of nibbles, looked up in the codebook with byte permutes
// Products use sdot4 (v_dot4_i32_i8); lane partials are reduced with cross-lane shuffles.
#include <map>
#include <mutex>
#include <stdlib.h>

#include "quant.hpp"

namespace hkhip {

constexpr int MV_PARTS = 4;
constexpr int MV_UNROLL = 4;                 // units per lane loaded before use
constexpr uint32_t MV_LDS_MAX = 160 * 1024;  // LDS per workgroup on gfx950

struct MvPart {
    const uint8_t *w;
    const uint16_t *ws; // scale plane (Q8_0, IQ4_NL, Q6_K)
    float *y;
    const float *bias;
    uint32_t rows;
    uint32_t row0; // first row of this part in the fused row space
};

struct MvArgs {
    MvPart p[MV_PARTS];
    uint32_t nparts, total_rows, K;
    const float *x;       // f32 input [NT][K], quantized in the prologue; or null
    const int8_t *gqs;    // pre-quantized input (engine activation buffer) when x is null
    const float *gd;
    const int16_t *gbs;
    int mode;
    int lpr_log2;
};

__device__ __forceinline__ uint4 ldw(const void *p) { return *reinterpret_cast<const uint4 *>(p); }

// LDS layout for NT tokens of K: qs [NT][K] i8 | bsums [NT][K/16] i16 (Q8K) | d [NT][K/blk] f32.
__host__ __device__ inline uint32_t mv_lds_bytes(int nt, uint32_t K, bool kq) {
    return nt * K + (kq ? nt * K / 8 : 0) + nt * (K / (kq ? 256 : 32)) * 4;
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
    const uint16_t *ws; // first scale of the row in the scale plane
};

// ---------------------------------------------------------------------------------------------
// Per-format unit load and unit dot. units(K) = work units per row.
// ---------------------------------------------------------------------------------------------

template <int T> struct MvFmt;

template <> struct MvFmt<HKHIP_Q4_K> {
    static constexpr bool kq = true;
    __device__ static uint32_t units(uint32_t K) { return K / 64; }
    struct W {
        uint4 h, q0, q1;
    };
    __device__ static RowRef row(const uint8_t *w, const uint16_t *, uint32_t r, uint32_t K) {
        return RowRef{w + uint64_t(r) * (K / 256) * 144, nullptr};
    }
    __device__ static W load(const RowRef &R, uint32_t u) {
        const uint8_t *blk = R.w + (u >> 2) * 144;
        return W{ldw(blk), ldw(blk + 16 + 32 * (u & 3)), ldw(blk + 32 + 32 * (u & 3))};
    }
    template <int NT>
    __device__ static void dot(const W &w, uint32_t u, const ActL &A, float *acc, float *corr) {
        const uint32_t sb = u >> 2, q = u & 3, K = A.K, nsb = K / 256;
        const uint4 h = w.h;
        // scalesMinsK4 word unpack (vecdot.zig:461-474), then sub-blocks 2q and 2q+1.
        const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
        const uint32_t mn_hi = ((h.w >> 4) & k2) | (((h.z >> 6) & k3) << 4);
        const uint32_t mn_lo = h.z & k1;
        const uint32_t sc_hi = (h.w & k2) | (((h.y >> 6) & k3) << 4);
        const uint32_t sc_lo = h.y & k1;
        const uint32_t sh = 16 * (q & 1);
        const uint32_t scw = ((q < 2) ? sc_lo : sc_hi) >> sh, mnw = ((q < 2) ? mn_lo : mn_hi) >> sh;
        const int sc0 = scw & 0xFF, sc1 = (scw >> 8) & 0xFF, mn0 = mnw & 0xFF, mn1 = (mnw >> 8) & 0xFF;
        const float d = f16_bits_to_f32(h.x & 0xFFFF), dmin = f16_bits_to_f32(h.x >> 16);
        const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int8_t *aq = A.qs + t * K + sb * 256 + 64 * q;
            const uint4 a0 = ldw(aq), a1 = ldw(aq + 16), a2 = ldw(aq + 32), a3 = ldw(aq + 48);
            const uint32_t aw[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                                     a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
            int slo = 0, shi = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                slo = sdot4(qw[i] & 0x0F0F0F0Fu, aw[i], slo);
                shi = sdot4((qw[i] >> 4) & 0x0F0F0F0Fu, aw[8 + i], shi);
            }
            const uint2 bsw = *reinterpret_cast<const uint2 *>(A.bs + t * (K / 16) + sb * 16 + 4 * q);
            const int b01 = int(int16_t(bsw.x & 0xFFFF)) + int(int16_t(bsw.x >> 16));
            const int b23 = int(int16_t(bsw.y & 0xFFFF)) + int(int16_t(bsw.y >> 16));
            const float ad = A.d[t * nsb + sb];
            acc[t] = fmaf((float)(slo * sc0 + shi * sc1), d * ad, acc[t]);
            corr[t] = fmaf((float)(mn0 * b01 + mn1 * b23), dmin * ad, corr[t]);
        }
    }
};

template <> struct MvFmt<HKHIP_Q6_K> {
    static constexpr bool kq = true;
    __device__ static uint32_t units(uint32_t K) { return K / 64; }
    struct W {
        uint4 l0, l1, hh;
        uint2 sc;
        uint32_t d;
    };
    __device__ static RowRef row(const uint8_t *w, const uint16_t *ws, uint32_t r, uint32_t K) {
        return RowRef{w + uint64_t(r) * (K / 256) * 208, ws + uint64_t(r) * (K / 256)};
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
    template <int NT>
    __device__ static void dot(const W &w, uint32_t u, const ActL &A, float *acc, float *) {
        const uint32_t sb = u >> 2, n = (u >> 1) & 1, lc = u & 1, K = A.K, nsb = K / 256;
        const int sc[4] = {int8_t(w.sc.x >> (8 * lc)), int8_t(w.sc.x >> (8 * lc + 16)),
                           int8_t(w.sc.y >> (8 * lc)), int8_t(w.sc.y >> (8 * lc + 16))};
        const uint32_t L0[4] = {w.l0.x, w.l0.y, w.l0.z, w.l0.w};
        const uint32_t L1[4] = {w.l1.x, w.l1.y, w.l1.z, w.l1.w};
        const uint32_t H[4] = {w.hh.x, w.hh.y, w.hh.z, w.hh.w};
        uint32_t qv[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            qv[0][i] = (L0[i] & 0x0F0F0F0Fu) | ((H[i] & 0x03030303u) << 4);
            qv[1][i] = (L1[i] & 0x0F0F0F0Fu) | (((H[i] >> 2) & 0x03030303u) << 4);
            qv[2][i] = ((L0[i] >> 4) & 0x0F0F0F0Fu) | (((H[i] >> 4) & 0x03030303u) << 4);
            qv[3][i] = ((L1[i] >> 4) & 0x0F0F0F0Fu) | (((H[i] >> 6) & 0x03030303u) << 4);
        }
        const float d = f16_bits_to_f32(w.d);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int8_t *aq = A.qs + t * K + sb * 256 + 128 * n + 16 * lc;
            const uint4 bsv = ldw(A.bs + t * (K / 16) + sb * 16 + 8 * n);
            const uint32_t bw[4] = {bsv.x, bsv.y, bsv.z, bsv.w};
            int isum = 0, bias = 0;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint4 av = ldw(aq + 32 * g);
                int s = sdot4(qv[g][0], av.x, 0);
                s = sdot4(qv[g][1], av.y, s);
                s = sdot4(qv[g][2], av.z, s);
                s = sdot4(qv[g][3], av.w, s);
                isum += s * sc[g];
                bias += sc[g] * int(int16_t(bw[g] >> (16 * lc)));
            }
            acc[t] = fmaf((float)(isum - 32 * bias), d * A.d[t * nsb + sb], acc[t]);
        }
    }
};

// Q8_0 and IQ4_NL: one 32-weight block per unit, against A8.
template <int T> struct MvLegacy {
    static constexpr bool kq = false;
    static constexpr uint32_t QB = (T == HKHIP_Q8_0) ? 32 : 16; // quant-plane bytes per block
    __device__ static uint32_t units(uint32_t K) { return K / 32; }
    struct W {
        uint4 x0, x1;
        uint32_t d;
    };
    __device__ static RowRef row(const uint8_t *w, const uint16_t *ws, uint32_t r, uint32_t K) {
        return RowRef{w + uint64_t(r) * (K / 32) * QB, ws + uint64_t(r) * (K / 32)};
    }
    __device__ static W load(const RowRef &R, uint32_t u) {
        W w;
        w.x0 = ldw(R.w + u * QB);
        if constexpr (T == HKHIP_Q8_0) w.x1 = ldw(R.w + u * QB + 16);
        w.d = R.ws[u];
        return w;
    }
    template <int NT>
    __device__ static void dot(const W &w, uint32_t u, const ActL &A, float *acc, float *) {
        uint32_t qw[8];
        if constexpr (T == HKHIP_Q8_0) {
            qw[0] = w.x0.x; qw[1] = w.x0.y; qw[2] = w.x0.z; qw[3] = w.x0.w;
            qw[4] = w.x1.x; qw[5] = w.x1.y; qw[6] = w.x1.z; qw[7] = w.x1.w;
        } else {
            const uint32_t n4[4] = {w.x0.x, w.x0.y, w.x0.z, w.x0.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                qw[i] = iq4nl_lookup4(n4[i] & 0x0F0F0F0Fu);
                qw[4 + i] = iq4nl_lookup4((n4[i] >> 4) & 0x0F0F0F0Fu);
            }
        }
        const float d = f16_bits_to_f32(w.d);
        const uint32_t K = A.K, U = K / 32;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int8_t *aq = A.qs + t * K + 32 * u;
            const uint4 a0 = ldw(aq), a1 = ldw(aq + 16);
            int s = sdot4(qw[0], a0.x, 0);
            s = sdot4(qw[1], a0.y, s);
            s = sdot4(qw[2], a0.z, s);
            s = sdot4(qw[3], a0.w, s);
            s = sdot4(qw[4], a1.x, s);
            s = sdot4(qw[5], a1.y, s);
            s = sdot4(qw[6], a1.z, s);
            s = sdot4(qw[7], a1.w, s);
            acc[t] = fmaf((float)s, d * A.d[t * U + u], acc[t]);
        }
    }
};
template <> struct MvFmt<HKHIP_Q8_0> : MvLegacy<HKHIP_Q8_0> {};
template <> struct MvFmt<HKHIP_IQ4_NL> : MvLegacy<HKHIP_IQ4_NL> {};

// ---------------------------------------------------------------------------------------------
// Kernel
// ---------------------------------------------------------------------------------------------

template <int T, int NT>
__global__ __launch_bounds__(256) void mmvq_kernel(MvArgs a) {
    using F = MvFmt<T>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr bool kq = F::kq;
    const uint32_t K = a.K;
    int8_t *sqs = reinterpret_cast<int8_t *>(smem);
    int16_t *sbs = reinterpret_cast<int16_t *>(smem + NT * K);
    float *sd = reinterpret_cast<float *>(smem + NT * K + (kq ? NT * K / 8 : 0));
    const ActL act{sqs, sbs, sd, K};
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t lg = a.lpr_log2, lpr = 1u << lg, rpw = 64u >> lg;
    const uint32_t sub = lane >> lg, ul = lane & (lpr - 1);
    const uint32_t groups = (a.total_rows + rpw - 1) / rpw;
    const uint32_t U = F::units(K);
    const uint32_t stride = gridDim.x * 4;

    // Row of this lane in group g: its part, local row and row pointers.
    auto locate = [&](uint32_t g, uint32_t &p, uint32_t &r, bool &active) -> RowRef {
        const uint32_t grow = g * rpw + sub;
        active = g < groups && grow < a.total_rows;
        p = 0;
#pragma unroll
        for (int i = 1; i < MV_PARTS; i++)
            if (i < int(a.nparts) && grow >= a.p[i].row0) p = i;
#define SEL(f) (p == 0 ? a.p[0].f : p == 1 ? a.p[1].f : p == 2 ? a.p[2].f : a.p[3].f)
        r = active ? grow - SEL(row0) : 0;
        return F::row(SEL(w), SEL(ws), r, K);
#undef SEL
    };

    typename F::W wv[MV_UNROLL];
    auto load_chunk = [&](const RowRef &R, bool active, uint32_t base) {
#pragma unroll
        for (int c = 0; c < MV_UNROLL; c++) {
            const uint32_t u = base + c * lpr;
            if (active && u < U) wv[c] = F::load(R, u);
        }
    };

    const uint32_t g0 = blockIdx.x * 4 + wave;
    uint32_t p, r;
    bool active;
    RowRef R = locate(g0, p, r, active);

    // Order of the memory traffic: the first batch of activation loads, then this wave's first
    // weight loads, then the activation work. Loads complete in issue order, so the activation
    // data can be used while the weight bytes are still in flight.
    constexpr int PB = 4; // activation loads per lane in the first batch
    float4 xv[PB];        // Q8K: one float4 of a block per lane
    float xs[PB];         // A8:  one value of a block per lane
    uint4 qv[PB];         // prepared input: 16 B of qs per thread
    if (a.x) {
        if constexpr (kq) {
            const uint32_t nblk = NT * K / 256;
#pragma unroll
            for (int j = 0; j < PB; j++) {
                const uint32_t b = wave + 4 * j;
                if (b < nblk) xv[j] = reinterpret_cast<const float4 *>(a.x + uint64_t(b) * 256)[lane];
            }
        } else {
            const uint32_t nblk = NT * K / 32, hw = tid >> 5, hl = tid & 31;
#pragma unroll
            for (int j = 0; j < PB; j++) {
                const uint32_t b = hw + 8 * j;
                xs[j] = b < nblk ? a.x[uint64_t(b) * 32 + hl] : 0.0f;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < PB; j++) {
            const uint32_t i = tid + 256 * j;
            if (i < NT * K / 16) qv[j] = reinterpret_cast<const uint4 *>(a.gqs)[i];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_chunk(R, active, ul);
    __builtin_amdgcn_sched_barrier(0);

    // ---- activations into LDS ----
#ifdef HKHIP_MV_PROBE_NO_PROLOGUE
    if (false) {
#else
    if (a.x) {
#endif
        if constexpr (kq) {
            const uint32_t nblk = NT * K / 256;
#pragma unroll
            for (int j = 0; j < PB; j++) {
                const uint32_t b = wave + 4 * j;
                if (b < nblk) {
                    const Q8KQ qr = quant_q8k_wave(xv[j], lane);
                    reinterpret_cast<uint32_t *>(sqs + b * 256)[lane] = qr.packed;
                    if ((lane & 3) == 0) sbs[b * 16 + lane / 4] = (int16_t)qr.bsum;
                    if (lane == 0) sd[b] = qr.d;
                }
            }
            for (uint32_t b = wave + 4 * PB; b < nblk; b += 4) {
                const Q8KQ qr = quant_q8k_wave(reinterpret_cast<const float4 *>(a.x + uint64_t(b) * 256)[lane], lane);
                reinterpret_cast<uint32_t *>(sqs + b * 256)[lane] = qr.packed;
                if ((lane & 3) == 0) sbs[b * 16 + lane / 4] = (int16_t)qr.bsum;
                if (lane == 0) sd[b] = qr.d;
            }
        } else {
            const uint32_t nblk = NT * K / 32, hw = tid >> 5, hl = tid & 31;
            // Both half-waves run every iteration (the quantizer needs the whole wave).
            const uint32_t nb2 = (nblk + 7) / 8 * 8;
#pragma unroll
            for (int j = 0; j < PB; j++) {
                const uint32_t b = hw + 8 * j;
                if (8 * j < nb2) {
                    const A8Q qr = quant_a8_halfwave(xs[j]);
                    if (b < nblk) {
                        sqs[b * 32 + hl] = (int8_t)qr.q;
                        if (hl == 0) sd[b] = qr.d;
                    }
                }
            }
            for (uint32_t b0 = 8 * PB; b0 < nb2; b0 += 8) {
                const uint32_t b = b0 + hw;
                const A8Q qr = quant_a8_halfwave(b < nblk ? a.x[uint64_t(b) * 32 + hl] : 0.0f);
                if (b < nblk) {
                    sqs[b * 32 + hl] = (int8_t)qr.q;
                    if (hl == 0) sd[b] = qr.d;
                }
            }
        }
    } else
#ifdef HKHIP_MV_PROBE_NO_PROLOGUE
    if (false)
#endif
    {
#pragma unroll
        for (int j = 0; j < PB; j++) {
            const uint32_t i = tid + 256 * j;
            if (i < NT * K / 16) reinterpret_cast<uint4 *>(sqs)[i] = qv[j];
        }
        for (uint32_t i = tid + 256 * PB; i < NT * K / 16; i += 256)
            reinterpret_cast<uint4 *>(sqs)[i] = reinterpret_cast<const uint4 *>(a.gqs)[i];
        const uint32_t nd = NT * (K / (kq ? 256 : 32));
        for (uint32_t i = tid; i < nd; i += 256) sd[i] = a.gd[i];
        if constexpr (kq)
            for (uint32_t i = tid; i < NT * K / 32; i += 256)
                reinterpret_cast<uint32_t *>(sbs)[i] = reinterpret_cast<const uint32_t *>(a.gbs)[i];
    }
#ifndef HKHIP_MV_PROBE_NO_PROLOGUE
    __syncthreads();
#endif

    // ---- rows ----
    for (uint32_t g = g0; g < groups; g += stride) {
        if (g != g0) {
            R = locate(g, p, r, active);
            load_chunk(R, active, ul);
        }
        float acc[NT], corr[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] = corr[t] = 0.0f;
        for (uint32_t base = ul; active && base < U;) {
#pragma unroll
            for (int c = 0; c < MV_UNROLL; c++) {
                const uint32_t u = base + c * lpr;
#ifdef HKHIP_MV_PROBE_LOADS_ONLY
                if (u < U) {
                    uint32_t xr = 0;
                    for (uint32_t i = 0; i < sizeof(wv[c]) / 4; i++) xr ^= reinterpret_cast<const uint32_t *>(&wv[c])[i];
                    acc[0] += __builtin_bit_cast(float, xr & 1u);
                }
#else
                if (u < U) F::template dot<NT>(wv[c], u, act, acc, corr);
#endif
            }
            base += MV_UNROLL * lpr;
            if (base < U) load_chunk(R, active, base);
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float v = acc[t] - corr[t];
            for (uint32_t off = lpr >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off);
            acc[t] = v;
        }
        if (active && ul == 0) {
            float *y = p == 0 ? a.p[0].y : p == 1 ? a.p[1].y : p == 2 ? a.p[2].y : a.p[3].y;
            const float *bias = p == 0 ? a.p[0].bias : p == 1 ? a.p[1].bias : p == 2 ? a.p[2].bias : a.p[3].bias;
            const uint32_t rows = p == 0 ? a.p[0].rows : p == 1 ? a.p[1].rows : p == 2 ? a.p[2].rows : a.p[3].rows;
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
    }
}

typedef void (*mv_kernel_t)(MvArgs);

template <int T>
static mv_kernel_t pick(int nt) {
    switch (nt) {
    case 1: return mmvq_kernel<T, 1>;
    case 2: return mmvq_kernel<T, 2>;
    case 3: return mmvq_kernel<T, 3>;
    case 4: return mmvq_kernel<T, 4>;
    case 5: return mmvq_kernel<T, 5>;
    case 6: return mmvq_kernel<T, 6>;
    case 7: return mmvq_kernel<T, 7>;
    case 8: return mmvq_kernel<T, 8>;
    default: return nullptr;
    }
}

static mv_kernel_t kernel_for(int t, int nt) {
    switch (t) {
    case HKHIP_Q4_K: return pick<HKHIP_Q4_K>(nt);
    case HKHIP_Q6_K: return pick<HKHIP_Q6_K>(nt);
    case HKHIP_Q8_0: return pick<HKHIP_Q8_0>(nt);
    case HKHIP_IQ4_NL: return pick<HKHIP_IQ4_NL>(nt);
    default: return nullptr;
    }
}

// Resident workgroups per CU for a kernel at an LDS size (cached; the first call per kernel also
// raises its dynamic-LDS limit to the full 160 KB).
static int resident_per_cu(mv_kernel_t k, uint32_t lds) {
    static std::mutex mu;
    static std::map<std::pair<void *, uint32_t>, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto key = std::make_pair(reinterpret_cast<void *>(k), lds);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                              int(MV_LDS_MAX));
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, 256, lds) != hipSuccess || n < 1) n = 1;
    cache[key] = n;
    return n;
}

static int cu_count() {
    static int n = 0;
    if (!n) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
    }
    return n;
}

static int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v ? atoi(v) : dflt;
}

hipError_t launch_mmvq_parts(int t, const MvPartDesc *parts, int nparts, uint32_t K, const float *x,
                             const uint8_t *xq, uint32_t n, int mode, hipStream_t s) {
    if (n < 1 || n > 8 || nparts < 1 || nparts > MV_PARTS) return hipErrorInvalidValue;
    const bool kq = (t == HKHIP_Q4_K || t == HKHIP_Q6_K);
    // Tokens per launch: as many as the LDS holds (all 8 at every BASELINE shape).
    int per = int(n);
    while (per > 1 && mv_lds_bytes(per, K, kq) > MV_LDS_MAX) per--;
    if (mv_lds_bytes(per, K, kq) > MV_LDS_MAX) return hipErrorInvalidValue;
    // Lanes per row: enough that each lane has MV_UNROLL units of the row in flight at once.
    const uint32_t units = kq ? K / 64 : K / 32;
    const uint32_t want_lanes = (units + MV_UNROLL - 1) / MV_UNROLL;
    int lg = 0;
    while ((1u << lg) < want_lanes && lg < 6) lg++;
    // Tuning overrides (experiments only): lanes-per-row log2, and the workgroup cap
    // (0 = one workgroup per 4 row groups, no persistence).
    static const int env_lg = env_int("HKHIP_MV_LPR", -1);
    static const int env_cap = env_int("HKHIP_MV_CAP", -1);
    if (env_lg >= 0 && env_lg <= 6) lg = env_lg;
    const ActLayout A = act_layout(n, K);
    const uint32_t dblk = kq ? 256 : 32;
    for (uint32_t t0 = 0; t0 < n; t0 += per) {
        const int nt = int(n - t0 < uint32_t(per) ? n - t0 : uint32_t(per));
        MvArgs a{};
        uint32_t total = 0;
        for (int i = 0; i < nparts; i++) {
            const WLayout W = weight_layout(t, parts[i].rows, K);
            a.p[i].w = parts[i].w;
            a.p[i].ws = reinterpret_cast<const uint16_t *>(parts[i].w + W.scale_off);
            a.p[i].y = parts[i].y + uint64_t(t0) * parts[i].rows;
            a.p[i].bias = parts[i].bias;
            a.p[i].rows = parts[i].rows;
            a.p[i].row0 = total;
            total += parts[i].rows;
        }
        for (int i = nparts; i < MV_PARTS; i++) a.p[i].row0 = 0xffffffffu;
        a.nparts = uint32_t(nparts);
        a.total_rows = total;
        a.K = K;
        a.mode = mode;
        a.lpr_log2 = lg;
        if (x) {
            a.x = x + uint64_t(t0) * K;
        } else {
            a.gqs = reinterpret_cast<const int8_t *>(xq + (kq ? A.k_qs : A.a8_qs)) + uint64_t(t0) * K;
            a.gd = reinterpret_cast<const float *>(xq + (kq ? A.k_d : A.a8_d)) + uint64_t(t0) * (K / dblk);
            a.gbs = reinterpret_cast<const int16_t *>(xq + A.k_bs) + uint64_t(t0) * (K / 16);
        }
        if (total == 0) continue;
        mv_kernel_t k = kernel_for(t, nt);
        if (!k) return hipErrorInvalidValue;
        const uint32_t lds = mv_lds_bytes(nt, K, kq);
        const uint32_t groups = (total + (64u >> lg) - 1) / (64u >> lg);
        const uint32_t want = (groups + 3) / 4;
        uint32_t cap = uint32_t(cu_count() * resident_per_cu(k, lds));
        if (env_cap == 0) cap = 0xffffffffu;
        else if (env_cap > 0) cap = uint32_t(env_cap);
        const uint32_t grid = want < cap ? want : cap;
        hipLaunchKernelGGL(k, dim3(grid), dim3(256), lds, s, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_mmvq(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n,
                       float *y, const float *bias, int mode, hipStream_t s) {
    MvPartDesc p{w, y, bias, rows};
    return launch_mmvq_parts(t, &p, 1, cols, nullptr, xq, n, mode, s);
}

} // namespace hkhip
