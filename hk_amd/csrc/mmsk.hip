// Small-batch product for Q4_K and Q6_K (4..32 tokens) on the int8 MFMA units.
//
// Between single-token decode and prefill the weights still dominate the bytes (each is used by
// a handful of tokens), so this kernel streams them like the decode kernels, but multiplies them
// against the tokens on v_mfma_i32_16x16x64_i8 instead of per-token dot products: the per-weight
// VALU work no longer grows with the token count.
//
// Arithmetic (hk's CPU kernel, src/quant/gemm.zig kernelK 180-236, per row r, token t,
// super-block b):  y += da*(d*I - dmin*J),  I = sum_s sc_s * sum_{k in s} q*a,
// J = sum_s mn_s * bsum32_s, both exact integers:
//  * I: the 6-bit scale is folded into the weights as two int8 planes, sc = 8*sh + sl, each
//    product at most 105 (one packed 16-bit multiply per four weights); the MFMA chain runs the
//    sh plane, the result is multiplied by 8, then the sl plane is added on top.
//  * J: one v_mfma_f32_16x16x32_bf16 over exact bf16 integers: the mins against the tokens'
//    bsum32 = 64*u + v (the activation buffer's k_ilmb plane), exact in f32 (|J| < 2^22).
// Q6_K (kernelK with the 16-weight groups): y += da*d*I, I = sum_g sc_g * sum_{k in g} (q - 32)*a.
// A lane's 16 weights of a chunk are one group, so the signed 8-bit scale folds into them,
// w = sc*(q - 32), split into two int8 planes 4*w = 256*H + L (H in [-63, 64], L in [-128, 124]);
// one int32 chain (H-sum << 8) + L-sum gives 4*I exactly (as the prefill GEMM).
//
// Layout. A workgroup owns 16 rows of one part (fused products: up to 4 matrices reading the
// same input, their row tiles numbered in sequence); its KS waves split the super-blocks and add
// their partial sums in LDS at the end. MFMA roles: A = weights (row = lane % 16), B =
// activations (token = lane % 16); lane group g = lane / 16 supplies values 16g..16g+15 of each
// 64-value chunk. Output lane l holds rows 4*(l/16) + i (i < 4) of token l % 16.
//
// Memory. Every global access is a contiguous piece of 1 KB (or 512 / 64 bytes): the weights of
// a super-block (16 rows x 144 bytes) go global -> LDS by direct loads into a per-wave ring of PF
// slots and are read back from there; the activations come from the token-interleaved planes
// the quantizer writes for small batches (k_il: a tile's 64-value chunk is 1 KB in lane order).
// The direct loads are issued as inline assembly (the compiler would otherwise wait for all of
// them before any LDS read it cannot prove independent) and waited for with an explicit count;
// the activation loads are ordinary, and the compiler's waits for them, which do not count the
// direct loads, keep about one super-block less in flight. The launches use PF = 2: fewer bytes
// in flight per wave, but twice the waves per SIMD of a deeper ring (see launch_mmsk_parts).
// Launches of up to 8 tokens and 256 or more four-tile workgroups take mmsa_kernel instead, whose
// workgroups stage the tokens' activations in LDS once rather than every wave re-reading them.

#include "common.hpp"

namespace hkhip {

// Helpers and the kernel live in a named namespace so that profiles show the kernel's name.
namespace sk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));

constexpr int SK_PARTS = 4;
// Quant-plane bytes of a row's super-block, and the 1-KB direct loads of a super-block for RT row
// tiles of 16 (Q6_K: 4 KB, of which 3328 bytes are the rows and 256 bytes after them the rows'
// scale words).
template <int T> constexpr uint32_t sk_rb() { return T == HKHIP_Q6_K ? 208 : 144; }
template <int T, int RT> constexpr uint32_t sk_dma() { return T == HKHIP_Q6_K ? 4 : (144 * 16 * RT + 1023) / 1024; }

struct SkPart {
    const uint8_t *w;
    const uint8_t *ws; // Q6_K: the f16 scale plane
    float *y;
    const float *bias;
    uint32_t rows, tile0; // tile0: first row tile of the part in the launch
};

struct SkArgs {
    SkPart p[SK_PARTS];
    uint32_t nparts, K, n, tiles; // tiles: 16-token tiles of the interleaved planes
    uint32_t rtiles;              // 16-row tiles of the launch (the shared-activation kernel)
    const uint8_t *il;
    const uint8_t *ilmb;
    const float *ild;
    int mode;
};

__device__ __forceinline__ uint32_t mul_bytes(uint32_t nib, uint32_t f2) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(us2, nib) * __builtin_bit_cast(us2, f2));
}

__device__ __forceinline__ v4i ld16(const void *g) { return *reinterpret_cast<const v4i *>(g); }

// s_waitcnt vmcnt(N), as assembly with a memory clobber so that no memory access (the LDS
// reads of the slot just waited for, in particular) moves across it.
template <int N> __device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// The activation operands of one super-block, per token tile.
template <int NTT> struct SkAct {
    v4i a[NTT][4];
    v4i mb[NTT];
    float da[NTT];
};

// One super-block of a 16-row tile against the token tiles of x (Q6_K). `slot` holds the rows'
// 208-byte blocks and, 3328 bytes in, the aligned words of their f16 scales; dodd picks the word's
// half.
template <int NTT>
__device__ __forceinline__ void sk_step_q6k(const uint8_t *slot, const SkAct<NTT> &x, float keep, uint32_t g,
                                            uint32_t p, uint32_t dodd, v4f (&acc)[1][NTT]) {
    // Lane (row p, group g), chunk c: values 64c + 16g.. = group 4c + g of the super-block,
    // i.e. ql bytes 64n + 32(g>>1) + 16(g&1).. (nibble c&1), qh bytes 128 + 32n + 16(g&1)..
    // (bits 2(2(c&1) + (g>>1))), scale byte 192 + 8n + 4(c&1) + 2(g>>1) + (g&1), n = c >> 1.
    const uint8_t *blk = slot + 208 * p;
    uint4 ql[2], qh[2];
#pragma unroll
    for (int n = 0; n < 2; n++) {
        ql[n] = *reinterpret_cast<const uint4 *>(blk + 64 * n + 32 * (g >> 1) + 16 * (g & 1));
        qh[n] = *reinterpret_cast<const uint4 *>(blk + 128 + 32 * n + 16 * (g & 1));
    }
    const uint4 scw = *reinterpret_cast<const uint4 *>(blk + 192);
    const uint32_t scs[4] = {scw.x, scw.y, scw.z, scw.w};
    const uint32_t dword = *reinterpret_cast<const uint32_t *>(slot + 16 * 208 + 4 * p);
    const float d = f16_bits_to_f32(dodd ? dword >> 16 : dword & 0xFFFF);
    // Planes H, L of the group-scaled weights (4*w = 256*H + L); 4*I is scaled by d/4.
    v4i P[2][4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int n = c >> 1;
        const uint32_t sidx = 8 * n + 4 * (c & 1) + 2 * (g >> 1) + (g & 1);
        const int sc = int(int8_t((scs[sidx / 4] >> (8 * (sidx % 4))) & 0xFF));
        const uint32_t m = q6k_m(sc), k = q6k_k(sc);
        const uint32_t qs = 2 * (2 * (c & 1) + (g >> 1));
        const uint32_t lw[4] = {ql[n].x, ql[n].y, ql[n].z, ql[n].w};
        const uint32_t hw[4] = {qh[n].x, qh[n].y, qh[n].z, qh[n].w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = ((lw[i] >> (4 * (c & 1))) & 0x0F0F0F0Fu) | (((hw[i] >> qs) & 0x03030303u) << 4);
            int hp, lp;
            q6k_planes(q, m, k, hp, lp);
            P[0][c][i] = hp;
            P[1][c][i] = lp;
        }
    }
    const float d4 = 0.25f * d;
    float dr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) dr[i] = __shfl(d4, int(4 * g + i));
#pragma unroll
    for (int tt = 0; tt < NTT; tt++) {
        v4i s = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 4; c++) s = __builtin_amdgcn_mfma_i32_16x16x64_i8(P[0][c], x.a[tt][c], s, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) s[i] <<= 8;
#pragma unroll
        for (int c = 0; c < 4; c++) s = __builtin_amdgcn_mfma_i32_16x16x64_i8(P[1][c], x.a[tt][c], s, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[0][tt][i] = fmaf((float)s[i], dr[i] * (x.da[tt] * keep), acc[0][tt][i]);
    }
}

// One super-block of RT 16-row tiles against the token tiles of x (Q4_K); `slot` holds the rows'
// 144-byte blocks.
template <int NTT, int RT>
__device__ __forceinline__ void sk_step_q4k(const uint8_t *slot, const SkAct<NTT> &x, float keep, uint32_t g,
                                            uint32_t p, v4f (&acc)[RT][NTT]) {
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const uint8_t *blk = slot + 144 * (16 * rt + p);
        const uint4 h = *reinterpret_cast<const uint4 *>(blk);
        uint4 q[4];
#pragma unroll
        for (int c = 0; c < 4; c++) q[c] = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * c + 16 * (g & 1));
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
            const uint32_t w4[4] = {q[c].x, q[c].y, q[c].z, q[c].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t nib = (w4[i] >> sh) & 0x0F0F0F0Fu;
                ph[c][i] = int(mul_bytes(nib, fh));
                pl[c][i] = int(mul_bytes(nib, fl));
            }
        }
        // Min-term A operand: the 8 mins as bf16 integers in lane groups 0 and 1, zero in 2, 3.
        uint32_t mw[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t src = i < 2 ? mnl : mnh, s = 16 * (i & 1);
            const float e = (float)((src >> s) & 0xFF), o = (float)((src >> (s + 8)) & 0xFF);
            mw[i] = g < 2 ? (__builtin_bit_cast(uint32_t, e) >> 16) | (__builtin_bit_cast(uint32_t, o) & 0xFFFF0000u) : 0u;
        }
        const v8bf am = __builtin_bit_cast(v8bf, make_uint4(mw[0], mw[1], mw[2], mw[3]));
        // Scales of this lane's output rows 4*(lane/16) + i, from the lanes that read them.
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
                s = __builtin_amdgcn_mfma_i32_16x16x64_i8(ph[c], x.a[tt][c], s, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) s[i] <<= 3;
#pragma unroll
            for (int c = 0; c < 4; c++)
                s = __builtin_amdgcn_mfma_i32_16x16x64_i8(pl[c], x.a[tt][c], s, 0, 0, 0);
            const v4i mbw = g < 2 ? x.mb[tt] : v4i{0, 0, 0, 0};
            const v4f j = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, __builtin_bit_cast(v8bf, mbw), v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[rt][tt][i] = fmaf(fmaf((float)s[i], dr[i], mr[i] * j[i]), x.da[tt] * keep, acc[rt][tt][i]);
        }
    }
}

// Stores the tiles of one wave: output lane l holds rows 4*(l/16) + i of token l % 16.
template <int NTT, int RT>
__device__ __forceinline__ void sk_store(const v4f (&acc)[RT][NTT], uint32_t n, int mode, uint32_t r0, uint32_t rows,
                                         float *Y, const float *B, uint32_t g, uint32_t p) {
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
#pragma unroll
        for (int tt = 0; tt < NTT; tt++) {
            const uint32_t tok = 16 * tt + p;
            if (tok < n && mode == HKHIP_SILU_MUL) {
                // Rows 4g + i of the tile: gate/up pairs (i = 0, 1) and (2, 3).
#pragma unroll
                for (int i = 0; i < 4; i += 2) {
                    const uint32_t r = r0 + 16 * rt + 4 * g + i;
                    if (r < rows) Y[uint64_t(tok) * (rows / 2) + r / 2] = silu_mul(acc[rt][tt][i], acc[rt][tt][i + 1]);
                }
            } else if (tok < n && (rows % 4) == 0 && (reinterpret_cast<uintptr_t>(Y) % 16) == 0 &&
                       r0 + 16 * rt + 4 * g + 3 < rows) {
                // The lane's four consecutive rows as one 16-byte store.
                const uint32_t r = r0 + 16 * rt + 4 * g;
                float4 *dst = reinterpret_cast<float4 *>(Y + uint64_t(tok) * rows + r);
                float4 v = make_float4(acc[rt][tt][0], acc[rt][tt][1], acc[rt][tt][2], acc[rt][tt][3]);
                if (B) {
                    v.x += B[r];
                    v.y += B[r + 1];
                    v.z += B[r + 2];
                    v.w += B[r + 3];
                }
                if (mode == HKHIP_ACCUMULATE) {
                    const float4 o = *dst;
                    v.x += o.x;
                    v.y += o.y;
                    v.z += o.z;
                    v.w += o.w;
                }
                *dst = v;
            } else if (tok < n) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t r = r0 + 16 * rt + 4 * g + i;
                    if (r < rows) {
                        float *dst = Y + uint64_t(tok) * rows + r;
                        const float v = acc[rt][tt][i] + (B ? B[r] : 0.0f);
                        if (mode == HKHIP_ACCUMULATE)
                            *dst += v;
                        else
                            *dst = v;
                    }
                }
            }
        }
    }
}

template <int T, int NTT, int KS, int PF, int RT>
__global__ __launch_bounds__(KS * 64) void mmsk_kernel(SkArgs a) {
    constexpr bool q6 = T == HKHIP_Q6_K;
    static_assert(!q6 || RT == 1, "Q6_K: one row tile per wave");
    constexpr uint32_t RB = sk_rb<T>(), NDMA = sk_dma<T, RT>(), SLOT = 1024 * NDMA;
    constexpr int OPS = NDMA + (q6 ? 1 : 0) + NTT * (q6 ? 5 : 6); // loads per super-block and wave
    __shared__ __attribute__((aligned(16))) uint8_t ring[KS][PF][SLOT];
    __shared__ v4f part[KS > 1 ? KS - 1 : 1][RT][NTT][64];

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t g = lane >> 4, p = lane & 15;
    const uint32_t nsb = a.K / 256;

    // Part and row tile of this workgroup (uniform). Fields are copied member by member so the
    // argument block is never indexed dynamically.
    uint32_t pi = 0;
#pragma unroll
    for (int i = 1; i < SK_PARTS; i++)
        if (i < int(a.nparts) && blockIdx.x >= a.p[i].tile0) pi = i;
    const uint8_t *W = a.p[0].w;
    const uint8_t *WS = a.p[0].ws;
    float *Y = a.p[0].y;
    const float *B = a.p[0].bias;
    uint32_t rows = a.p[0].rows, tile0 = a.p[0].tile0;
#pragma unroll
    for (int i = 1; i < SK_PARTS; i++) {
        if (pi == uint32_t(i)) {
            W = a.p[i].w;
            WS = a.p[i].ws;
            Y = a.p[i].y;
            B = a.p[i].bias;
            rows = a.p[i].rows;
            tile0 = a.p[i].tile0;
        }
    }
    const uint32_t r0 = (blockIdx.x - tile0) * 16 * RT;
    const uint32_t sb0 = nsb * wave / KS, sb1 = nsb * (wave + 1) / KS;

    // Weight piece P = 64i + lane (16 bytes) of a super-block: byte 16*(P % PPR) of row P / PPR's
    // block; pieces past the last repeat it (they land in the slot's padding). Q6_K's scale words
    // sit right after the rows, where the last load's padding lanes would write: those lanes are
    // switched off (two direct loads into the same LDS bytes land in no defined order).
    constexpr uint32_t PPR = RB / 16, NP = PPR * 16 * RT;
    uint32_t woff[NDMA];
#pragma unroll
    for (uint32_t i = 0; i < NDMA; i++) {
        const uint32_t P = 64 * i + lane < NP ? 64 * i + lane : NP - 1;
        const uint32_t row = r0 + P / PPR < rows ? r0 + P / PPR : rows - 1;
        woff[i] = row * nsb * RB + 16 * (P % PPR);
    }
    // Q6_K scales: lane L loads the aligned word holding row r0 + L % 16's f16 for the super-block.
    const uint32_t srow = r0 + (lane & 15) < rows ? r0 + (lane & 15) : rows - 1;
    const uint32_t sbase = srow * nsb;
    uint8_t (*const myring)[SLOT] = ring[wave];

    // Lanes of tokens past n read the last token's entries: the same addresses as its own lanes,
    // so a load brings in only the real tokens' bytes.
    uint32_t tp[NTT];
#pragma unroll
    for (int tt = 0; tt < NTT; tt++) tp[tt] = 16 * tt + p < a.n ? p : a.n - 1 - 16 * tt;
    auto issue = [&](uint32_t sb, uint8_t *slot, SkAct<NTT> &x) {
        const uint8_t *gw = W + uint64_t(sb) * RB;
#pragma unroll
        for (uint32_t i = 0; i < NDMA; i++)
            if (!q6 || 64 * i + lane < NP) load_lds16(gw + woff[i], slot + 1024 * i);
        if constexpr (q6) load_lds4(WS + (((sbase + sb) >> 1) << 2), slot + 16 * RB);
#pragma unroll
        for (int tt = 0; tt < NTT; tt++) {
            const uint8_t *ga = a.il + ((uint64_t(4 * sb) * a.tiles + tt) * 64 + 16 * g + tp[tt]) * 16;
#pragma unroll
            for (int c = 0; c < 4; c++) x.a[tt][c] = ld16(ga + uint64_t(c) * a.tiles * 1024);
            if constexpr (!q6) x.mb[tt] = ld16(a.ilmb + ((uint64_t(sb) * a.tiles + tt) * 2 + (g & 1)) * 256 + 16 * tp[tt]);
            x.da[tt] = a.ild[(uint64_t(sb) * a.tiles + tt) * 16 + tp[tt]];
        }
    };

    v4f acc[RT][NTT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int tt = 0; tt < NTT; tt++) acc[rt][tt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    if (sb0 < sb1) {
        SkAct<NTT> x[PF];
        const uint32_t last = sb1 - 1;
        // PF-1 super-blocks in flight ahead of the one computed. Every step issues the same loads
        // (past the wave's range, repeats of its last super-block, multiplied by zero), so one
        // wait count fits all.
#pragma unroll
        for (int i = 0; i < PF - 1; i++) issue(sb0 + i < last ? sb0 + i : last, myring[i], x[i]);
        for (uint32_t sb = sb0; sb <= last; sb += PF) {
#pragma unroll
            for (int i = 0; i < PF; i++) {
                const uint32_t nx = sb + i + PF - 1;
                issue(nx < last ? nx : last, myring[(i + PF - 1) % PF], x[(i + PF - 1) % PF]);
                wait_vm<OPS * (PF - 1)>();
                const float keep = sb + i <= last ? 1.0f : 0.0f;
                if constexpr (q6)
                    sk_step_q6k<NTT>(myring[i], x[i], keep, g, p, (sbase + (sb + i <= last ? sb + i : last)) & 1, acc);
                else
                    sk_step_q4k<NTT, RT>(myring[i], x[i], keep, g, p, acc);
            }
        }
        wait_vm<0>(); // nothing in flight past the loop
    }

    // Partial sums of the waves meet in LDS; wave 0 finishes the rows.
    if (wave > 0) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int tt = 0; tt < NTT; tt++) part[wave - 1][rt][tt][lane] = acc[rt][tt];
    }
    if (KS > 1) __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int tt = 0; tt < NTT; tt++)
#pragma unroll
                for (int w = 0; w < KS - 1; w++) acc[rt][tt] += part[w][rt][tt][lane];
        sk_store<NTT, RT>(acc, a.n, a.mode, r0, rows, Y, B, g, p);
    }
}


// ---- Shared-activation variant (at most SA_TOK tokens, one token tile) ----
//
// Each wave above re-reads a super-block's activation operands from L2 for every 16-row tile
// (5.3 KB against the tile's 2.3 KB of weights), and those reads, not the weights, set its rate
// (a loads-only probe of that structure: 20.1 us for 66 MB, against 13.1 us for the weights
// alone). Here a workgroup of SA_NR waves, each with its own 16-row tile over the whole K, first
// copies the live tokens' interleaved entries (k_il / k_ilmb / k_ild, tokens 0..SA_TOK-1 of tile
// 0) into LDS by direct loads, behind one barrier; afterwards a wave's only global loads are its
// weights, through the same two-slot ring, and the activation operands come from LDS (the probe
// of this structure: 14.7 us). Measured at 8 tokens on Llama-3-8B shapes, alternating runs against
// the kernel above: the batch-8 decode step 1.97-2.04 vs 2.09-2.10 ms, gate/up 21.4-22.4 vs
// 21.6-23.9 us; a ring of three or four slots (no register cost here) was slower, 23.4-23.9 us.
// Four tiles per workgroup: two (twice the staging, three workgroups per CU) took gate/up to 28.4
// us and the Q6_K lm_head to 121 us (vs 21.3 / 101.7); eight, 23.4 (the old kernel: too few
// workgroups) / 106.9.
constexpr uint32_t SA_NR = 4, SA_TOK = 8, SA_PF = 2;

// LDS geometry: A [nsb*4 chunks][4 g][SA_TOK] x 16 B, MB [nsb][2][SA_TOK] x 16 B (Q4_K),
// D [nsb][SA_TOK] f32, then the waves' rings; each staged region padded to whole direct loads.
struct SaGeom {
    uint32_t la, lm, ld; // direct loads of each region (1 KB, 1 KB, 256 B)
    uint32_t mb, d, ring, total;
};
template <int T> __host__ __device__ inline SaGeom sa_geom(uint32_t nsb) {
    SaGeom G{};
    G.la = nsb * 16 * SA_TOK / 64;
    G.lm = T == HKHIP_Q6_K ? 0 : (nsb * 2 * SA_TOK + 63) / 64;
    G.ld = (nsb * SA_TOK + 63) / 64;
    G.mb = 1024 * G.la;
    G.d = G.mb + 1024 * G.lm;
    G.ring = G.d + 256 * G.ld;
    G.total = G.ring + SA_NR * SA_PF * 1024 * sk_dma<T, 1>();
    return G;
}

template <int T>
__global__ __launch_bounds__(SA_NR * 64) void mmsa_kernel(SkArgs a) {
    constexpr bool q6 = T == HKHIP_Q6_K;
    constexpr uint32_t RB = sk_rb<T>(), NDMA = sk_dma<T, 1>(), SLOT = 1024 * NDMA;
    constexpr int OPS = NDMA + (q6 ? 1 : 0); // loads per super-block and wave
    extern __shared__ __attribute__((aligned(16))) uint8_t sa_smem[];

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t g = lane >> 4, p = lane & 15;
    const uint32_t nsb = a.K / 256, last = nsb - 1;
    const SaGeom G = sa_geom<T>(nsb);
    uint8_t *const A = sa_smem;
    uint8_t *const MB = sa_smem + G.mb;
    uint8_t *const D = sa_smem + G.d;
    uint8_t *const ring = sa_smem + G.ring + wave * SA_PF * SLOT;

    // This wave's row tile and its part (wave-uniform); waves past the last tile stage and wait
    // with the others, then stream the last tile again and store nothing.
    const uint32_t tile_raw = blockIdx.x * SA_NR + wave;
    const bool real = tile_raw < a.rtiles;
    const uint32_t tile = real ? tile_raw : a.rtiles - 1;
    uint32_t pi = 0;
#pragma unroll
    for (int i = 1; i < SK_PARTS; i++)
        if (i < int(a.nparts) && tile >= a.p[i].tile0) pi = i;
    const uint8_t *W = a.p[0].w;
    const uint8_t *WS = a.p[0].ws;
    float *Y = a.p[0].y;
    const float *B = a.p[0].bias;
    uint32_t rows = a.p[0].rows, tile0 = a.p[0].tile0;
#pragma unroll
    for (int i = 1; i < SK_PARTS; i++) {
        if (pi == uint32_t(i)) {
            W = a.p[i].w;
            WS = a.p[i].ws;
            Y = a.p[i].y;
            B = a.p[i].bias;
            rows = a.p[i].rows;
            tile0 = a.p[i].tile0;
        }
    }
    const uint32_t r0 = (tile - tile0) * 16;

    constexpr uint32_t PPR = RB / 16, NP = PPR * 16;
    uint32_t woff[NDMA];
#pragma unroll
    for (uint32_t i = 0; i < NDMA; i++) {
        const uint32_t P = 64 * i + lane < NP ? 64 * i + lane : NP - 1;
        const uint32_t row = r0 + P / PPR < rows ? r0 + P / PPR : rows - 1;
        woff[i] = row * nsb * RB + 16 * (P % PPR);
    }
    const uint32_t srow = r0 + (lane & 15) < rows ? r0 + (lane & 15) : rows - 1;
    const uint32_t sbase = srow * nsb;
    auto issue = [&](uint32_t sb, uint8_t *slot) {
        const uint8_t *gw = W + uint64_t(sb) * RB;
#pragma unroll
        for (uint32_t i = 0; i < NDMA; i++)
            if (!q6 || 64 * i + lane < NP) load_lds16(gw + woff[i], slot + 1024 * i);
        if constexpr (q6) load_lds4(WS + (((sbase + sb) >> 1) << 2), slot + 16 * RB);
    };
#pragma unroll
    for (uint32_t i = 0; i + 1 < SA_PF; i++) issue(i < last ? i : last, ring + SLOT * i);

    // Staging: direct load i of a region goes to wave i % SA_NR; entry q = 64*i + lane. Tokens
    // past n take the last token's entries (never read: padding lanes read that token's own).
    const uint32_t nt = a.n;
    auto tok = [&](uint32_t q) { const uint32_t t = q % SA_TOK; return t < nt ? t : nt - 1; };
    for (uint32_t i = wave; i < G.la; i += SA_NR) {
        const uint32_t q = 64 * i + lane, gq = (q / SA_TOK) % 4, ch = q / (4 * SA_TOK);
        load_lds16(a.il + (uint64_t(ch) * a.tiles * 64 + 16 * gq + tok(q)) * 16, A + 1024 * i);
    }
    if constexpr (!q6) {
        for (uint32_t i = wave; i < G.lm; i += SA_NR) {
            const uint32_t q = 64 * i + lane, h1 = (q / SA_TOK) % 2;
            const uint32_t sb = q / (2 * SA_TOK) < nsb ? q / (2 * SA_TOK) : last;
            load_lds16(a.ilmb + ((uint64_t(sb) * a.tiles) * 2 + h1) * 256 + 16 * tok(q), MB + 1024 * i);
        }
    }
    for (uint32_t i = wave; i < G.ld; i += SA_NR) {
        const uint32_t q = 64 * i + lane;
        const uint32_t sb = q / SA_TOK < nsb ? q / SA_TOK : last;
        load_lds4(a.ild + (uint64_t(sb) * a.tiles) * 16 + tok(q), D + 256 * i);
    }
    wait_vm<0>();
    __syncthreads();

    const uint32_t tpc = p < nt ? p : nt - 1;
    auto fetch = [&](uint32_t sb, SkAct<1> &x) {
#pragma unroll
        for (int c = 0; c < 4; c++)
            x.a[0][c] = *reinterpret_cast<const v4i *>(A + (((4 * sb + c) * 4 + g) * SA_TOK + tpc) * 16);
        if constexpr (!q6) x.mb[0] = *reinterpret_cast<const v4i *>(MB + ((sb * 2 + (g & 1)) * SA_TOK + tpc) * 16);
        x.da[0] = *reinterpret_cast<const float *>(D + (sb * SA_TOK + tpc) * 4);
    };

    v4f acc[1][1] = {{v4f{0.0f, 0.0f, 0.0f, 0.0f}}};
    for (uint32_t sb = 0; sb <= last; sb += SA_PF) {
#pragma unroll
        for (uint32_t i = 0; i < SA_PF; i++) {
            const uint32_t nx = sb + i + SA_PF - 1;
            issue(nx < last ? nx : last, ring + SLOT * ((i + SA_PF - 1) % SA_PF));
            wait_vm<OPS * (SA_PF - 1)>();
            const uint32_t cur = sb + i <= last ? sb + i : last;
            SkAct<1> x;
            fetch(cur, x);
            const float keep = sb + i <= last ? 1.0f : 0.0f;
            if constexpr (q6)
                sk_step_q6k<1>(ring + SLOT * i, x, keep, g, p, (sbase + cur) & 1, acc);
            else
                sk_step_q4k<1, 1>(ring + SLOT * i, x, keep, g, p, acc);
        }
    }
    wait_vm<0>();
    if (real) sk_store<1, 1>(acc, a.n, a.mode, r0, rows, Y, B, g, p);
}

typedef void (*sk_kernel_t)(SkArgs);

// At most 4 waves with two row tiles each (the LDS ring of 8 would not fit).
template <int RT> constexpr uint32_t sk_max_ks() { return RT > 1 ? 4 : 8; }
template <int T, int NTT, int PF, int RT> sk_kernel_t sk_pick(uint32_t ks) {
    if constexpr (sk_max_ks<RT>() >= 8)
        if (ks == 8) return mmsk_kernel<T, NTT, 8, PF, RT>;
    return ks == 1 ? mmsk_kernel<T, NTT, 1, PF, RT>
         : ks == 2 ? mmsk_kernel<T, NTT, 2, PF, RT>
                   : mmsk_kernel<T, NTT, 4, PF, RT>;
}

} // namespace sk

using sk::SkArgs;
using sk::SkPart;
using sk::sk_kernel_t;
using sk::sk_pick;
using sk::sk_max_ks;
using sk::SK_PARTS;

bool mmsk_supports(int t, uint32_t rows, uint32_t cols, uint32_t n) {
    // 32-bit per-lane offsets into the quant plane (and, Q6_K, the scale plane after it).
    return (t == HKHIP_Q4_K || t == HKHIP_Q6_K) && cols % 256 == 0 && rows > 0 && n >= 1 && n <= SK_MAX_TOKENS &&
           weight_layout(t, rows, cols).total < (1ull << 32);
}

hipError_t launch_mmsk_parts(int t, const MvPartDesc *parts, int nparts, uint32_t cols, const uint8_t *xq,
                             uint32_t n, int mode, hipStream_t s) {
    if (nparts < 1 || nparts > SK_PARTS) return hipErrorInvalidValue;
    for (int i = 0; i < nparts; i++)
        if (!mmsk_supports(t, parts[i].rows, cols, n)) return hipErrorInvalidValue;
    const ActLayout A = act_layout(n, cols);
    if (A.tiles == 0) return hipErrorInvalidValue;
    // Row tiles of 16 per wave: 1 (two share the activation loads, but need 320 VGPRs and
    // measured slower).
    constexpr uint32_t RT = 1;
    SkArgs a{};
    uint32_t tiles = 0;
    for (int i = 0; i < nparts; i++) {
        a.p[i] = SkPart{parts[i].w, parts[i].w + weight_layout(t, parts[i].rows, cols).scale_off, parts[i].y,
                        parts[i].bias, parts[i].rows, tiles};
        tiles += (parts[i].rows + 16 * RT - 1) / (16 * RT);
    }
    for (int i = nparts; i < SK_PARTS; i++) a.p[i].tile0 = 0xffffffffu;
    a.nparts = uint32_t(nparts);
    a.K = cols;
    a.n = n;
    a.tiles = A.tiles;
    a.il = xq + A.k_il;
    a.ilmb = xq + A.k_ilmb;
    a.ild = reinterpret_cast<const float *>(xq + A.k_ild);
    a.mode = mode;
    // K slices: enough waves for ~2048 in the launch, each with at least 2 super-blocks when the
    // matrix has them. (At least 4, as first set, left Qwen3-0.6B's products at 8 tokens on 64-384
    // workgroups of one or two waves: 8 sequences per pass 1.49-1.51 vs 1.34-1.36 ms; the Llama-3-8B
    // pass and batch-8 step measured the same either way, 2.51-2.53 and 2.03-2.13 ms.)
    const uint32_t nsb = cols / 256;
    uint32_t ks = 1;
    // (More waves, K slices up to 4096 or 8192 in the launch: the Llama-3-8B 8-sequence pass 2.57-2.62
    // vs 2.52 ms.)
    while (ks < sk_max_ks<RT>() && tiles * ks * 2 <= 2048 && nsb / (2 * ks) >= 2) ks *= 2;
    // Up to SA_TOK tokens, a launch of at least 256 shared-activation workgroups whose staged
    // activations leave room for two workgroups per CU: that kernel.
    if (n <= sk::SA_TOK && (tiles + sk::SA_NR - 1) / sk::SA_NR >= 256) {
        const uint32_t lds = t == HKHIP_Q6_K ? sk::sa_geom<HKHIP_Q6_K>(nsb).total : sk::sa_geom<HKHIP_Q4_K>(nsb).total;
        if (lds <= 80u * 1024) {
            const sk_kernel_t k = t == HKHIP_Q6_K ? sk::mmsa_kernel<HKHIP_Q6_K> : sk::mmsa_kernel<HKHIP_Q4_K>;
            static bool attr[2] = {false, false};
            if (!attr[t == HKHIP_Q6_K]) {
                (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                          int(80u * 1024));
                attr[t == HKHIP_Q6_K] = true;
            }
            a.rtiles = tiles;
            hipLaunchKernelGGL(k, dim3((tiles + sk::SA_NR - 1) / sk::SA_NR), dim3(sk::SA_NR * 64), lds, s, a);
            return hipGetLastError();
        }
    }
    // A ring of two slots: one super-block in flight while the other is computed. Deeper rings keep
    // more bytes in flight per wave but need more registers for the activations, which halves
    // the waves per SIMD (Q4_K, 16 tokens: 116 VGPRs and four waves at two slots, 192 and two at
    // four); measured at 8 tokens on Llama-3-8B shapes, two slots against four: q/k/v 8.5 vs 10.2 us,
    // o 6.6 vs 7.0, gate/up 22.8 vs 23.6, down 14.4 vs 16.0, the Q6_K lm_head 126 vs 145; at 32
    // tokens gate/up 31.2 vs 36.6 (three slots), lm_head 158 vs 182.
    const sk_kernel_t k = t == HKHIP_Q6_K ? (A.tiles == 1 ? sk_pick<HKHIP_Q6_K, 1, 2, RT>(ks) : sk_pick<HKHIP_Q6_K, 2, 2, RT>(ks))
                                          : (A.tiles == 1 ? sk_pick<HKHIP_Q4_K, 1, 2, RT>(ks) : sk_pick<HKHIP_Q4_K, 2, 2, RT>(ks));
    hipLaunchKernelGGL(k, dim3(tiles), dim3(ks * 64), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_mmsk(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n,
                       float *y, const float *bias, int mode, hipStream_t s) {
    const MvPartDesc p{w, y, bias, rows};
    return launch_mmsk_parts(t, &p, 1, cols, xq, n, mode, s);
}

} // namespace hkhip
