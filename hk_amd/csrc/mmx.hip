// Prefill GEMM for Q6_K and the 32-weight formats (Q8_0, IQ4_NL, Q4_0, Q4_1, Q5_0, Q5_1) on the
// int8 MFMA units (K a multiple of 256).
//
// Integer arithmetic as in hk's CPU kernels (src/quant/gemm.zig kernelK 180-236 for Q6_K,
// kernelLegacy 131-176 for the 32-weight blocks):
//  * Q6_K: per row r, token t and super-block b, y += d[r,b]*da[t,b] * I with the exact integer
//    I = sum_g sc[r,b,g] * sum_{k in g} (q[r,k] - 32) * a[t,k] over the 16 groups of 16. The
//    signed 8-bit group scale is folded into the weights, w = sc*(q - 32) in [-4096, 4096], and
//    w is split into two int8 planes, 4*w = 256*H + L with H in [-63, 64] and L in [-128, 124].
//    Each MFMA lane holds 16 weights of one group (one scale per lane and chunk). One int32
//    chain per tile gives (H-sum << 8) + L-sum = 4*I, the reference's integer times four.
//  * 32-weight formats: y += (dw[r,c]*da[t,c]) * I_c per block c (I_c exact). One 32x32x32
//    int8 MFMA yields the tile's I_c; then per output one multiply (dw*da), one convert and one
//    fma. Q4_0 / Q5_0 weights enter as u - zp (kernelLegacy's acci - zp*s); Q4_1 / Q5_1 as u,
//    plus m[r,c] * (da[t,c] * s[t,c]) per output (kernelLegacy's has_m term; the product comes
//    precomputed from qact).
// Only the f32 summation order differs from the reference.
//
// Structure (as the Q4_K ring kernel): a workgroup of NW waves owns 32*NW rows x 32*TT tokens;
// every operand of a super-block (256 weights) goes global -> LDS by direct loads into a ring of
// NB slots, NB-1 super-blocks ahead of the compute; each lane builds its row's MFMA operands
// from LDS. MFMA roles: A = activations (tokens as M), B = weights (rows as N); output lane l
// holds row l%32 and tokens 8*(v/4) + 4*(l/32) + v%4.

#include "common.hpp"
#include "gemm_store.hpp"

#include <type_traits>

namespace hkhip {
namespace mx {

typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// Per-format geometry of one super-block step (256 weights of 32 rows = one wave's share).
template <int T> struct Fmt;
template <> struct Fmt<HKHIP_Q6_K> {
    static constexpr uint32_t RB = 208;  // quant-plane bytes per row and step
    static constexpr uint32_t W16 = 6;   // 1-KB direct loads per wave
    static constexpr uint32_t W4 = 2;    // 256-B direct loads (the rest)
    static constexpr uint32_t WSB = 256; // scale bytes per wave (one dword per lane)
    static constexpr uint32_t DAB = 4;   // activation-scale bytes per token and step
};
template <> struct Fmt<HKHIP_Q8_0> {
    static constexpr uint32_t RB = 256, W16 = 8, W4 = 0, WSB = 1024, DAB = 32;
};
template <> struct Fmt<HKHIP_IQ4_NL> {
    static constexpr uint32_t RB = 128, W16 = 4, W4 = 0, WSB = 1024, DAB = 32;
};
// Q4_0..Q5_1: side data per row and step: d (16 B) and m (16 B) as one 1-KB load per wave (lanes
// 32-63 take m), the fifth-bit words (32 B) as a second.
template <int T> struct Fmt4 {
    static constexpr uint32_t RB = 128, W16 = 4, W4 = 0, WSB = has_qh(T) ? 2048 : 1024, DAB = 32;
};
// IQ4_XS: IQ4_NL's 16 B per 32 weights; the 8-B block header (d, scales_h, scales_l) per row and
// step as one 4-B load per lane (lane L: row L/2's word L%2).
template <> struct Fmt<HKHIP_IQ4_XS> {
    static constexpr uint32_t RB = 128, W16 = 4, W4 = 0, WSB = 256, DAB = 4;
};
// Q5_K: hk's 176-B blocks as they are (header, qh[32], qs[128]); rows unswizzled like Q6_K's.
template <> struct Fmt<HKHIP_Q5_K> {
    static constexpr uint32_t RB = 176, W16 = 5, W4 = 2, WSB = 16, DAB = 4;
};
template <> struct Fmt<HKHIP_Q4_0> : Fmt4<HKHIP_Q4_0> {};
template <> struct Fmt<HKHIP_Q4_1> : Fmt4<HKHIP_Q4_1> {};
template <> struct Fmt<HKHIP_Q5_0> : Fmt4<HKHIP_Q5_0> {};
template <> struct Fmt<HKHIP_Q5_1> : Fmt4<HKHIP_Q5_1> {};

// MF: the Q4_1 / Q5_1 offset term on MFMAs (the single-slice tiles); with K slices the ring has
// no room for its operand and the term is one fma per output and block.
template <int T, int TOK, int NW, bool MF = true> struct MxSlot {
    int8_t a[TOK * 256];                     // chunk c of token t at c ^ (t & 15)
    uint8_t w[NW][32 * Fmt<T>::RB];          // per wave, its 32 rows' bytes of the step
    uint8_t ws[NW][Fmt<T>::WSB];             // per wave, the rows' f16 scales of the step
    // Activation scales: Q6_K per token (wave m fills tokens 64m..64m+63); A8 per block and token,
    // block-major ([8][TOK]), so that four consecutive tokens' scales are one 16-byte read.
    float da[T == HKHIP_Q6_K || T == HKHIP_IQ4_XS || T == HKHIP_Q5_K ? 64 * NW : 8 * TOK];
    // Q5_K: each sub-block's d_a * bsum32; Q4_1 / Q5_1 without MF: the blocks' d_a * s (f32
    // bits, [8][TOK] as da).
    uint32_t sa[T == HKHIP_Q5_K || (has_m(T) && !MF) ? 8 * TOK : 1];
    // Q4_1 / Q5_1: the blocks' d_a * s as three bf16 parts, [token][part][8] (a8_dsb), in 1-KB
    // chunks, one load per wave (waves past the last chunk load it again).
    uint32_t dsb[has_m(T) && MF ? 256 * ((TOK * 48 + 1023) / 1024) : 0];
};

struct MxArgs {
    const uint8_t *w;
    const uint8_t *ws; // f16 scale plane
    uint32_t rows, cols, n;
    const int8_t *aqs;
    const float *ad;
    const float *ads;    // A8 d * s per block (Q4_1, Q5_1)
    const uint8_t *adsb; // the same in bf16 parts, [k/256][n][48 B]
    const float *adb;   // Q8K d * bsum32 per sub-block (Q5_K)
    float *y;
    const float *bias;
    int mode;
    int wide; // y 16-byte aligned and rows a multiple of 4: whole tiles go out as 16-byte stores
    uint32_t rblocks, tblocks;
};


// KS > 1 splits K over KS slices of NW waves, each with its own ring; the partial tiles are
// added in LDS in slice order at the end (as in the Q4_K ring kernel).
template <int T, int NW, int TT, int NB, int KS = 1>
__global__ __launch_bounds__(NW * KS * 64, 1) void mmx_kernel(MxArgs a) {
    constexpr int TOK = 32 * TT;
    using F = Fmt<T>;
    constexpr bool mf = has_m(T) && KS == 1; // offset term on MFMAs
    using Slot = MxSlot<T, TOK, NW, KS == 1>;
    constexpr bool q6 = (T == HKHIP_Q6_K);
    constexpr bool xs = (T == HKHIP_IQ4_XS);
    constexpr bool k5 = (T == HKHIP_Q5_K);
    constexpr bool kqa = q6 || xs || k5; // Q8K activations: one scale per token and super-block
    constexpr bool unswz = q6 || k5;     // rows not a power of two of pieces: no swizzle, word tail
    constexpr uint32_t DBS = 8 * TOK / (64 * NW); // Q5_K: bsum-pair loads per wave
    static_assert(NB == 2 || NB == 3, "ring depth");
    static_assert(kqa ? TOK <= 64 * NW : (8 * TOK) % (64 * NW) == 0, "token scales per wave");
    __shared__ __attribute__((aligned(16))) Slot ring0[KS];
    __shared__ __attribute__((aligned(16))) Slot ring1[KS];
    __shared__ __attribute__((aligned(16))) Slot ring2[KS];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wall = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t ks = wall / NW, wave = wall % NW; // K slice, row wave within the slice
    auto slot_at = [&](auto ic) -> Slot & {
        constexpr int i = decltype(ic)::value;
        if constexpr (i == 0)
            return ring0[ks];
        else if constexpr (i == 1)
            return ring1[ks];
        else
            return ring2[ks];
    };
    const uint32_t h = lane >> 5, j = lane & 31;
    const uint32_t K = a.cols, nsb = K / 256;

    // Workgroup -> (row block, token block); the token blocks of a row block run on one XCD so
    // its L2 serves the repeated weight reads (workgroups go round-robin over the 8 XCDs).
    uint32_t rb, tb;
    {
        const uint32_t i = blockIdx.x;
        if (a.rblocks % 8 == 0) {
            const uint32_t xcd = i % 8, k = i / 8;
            rb = xcd * (a.rblocks / 8) + k / a.tblocks;
            tb = k % a.tblocks;
        } else {
            rb = i / a.tblocks;
            tb = i % a.tblocks;
        }
    }
    const uint32_t r0 = rb * 32 * NW, t0 = tb * TOK;
    const uint32_t myrow = r0 + 32 * wave + j;
    auto clamp_row = [&](uint32_t r) { return r < a.rows ? r : a.rows - 1; };
    auto clamp_tok = [&](uint32_t t) { return t < a.n ? t : a.n - 1; };

    // ---- per-lane 32-bit offsets of the direct loads (mmx_supports checks that they fit) ----
    constexpr uint32_t TPW = TOK / NW; // token rows per wave
    static_assert(TPW % 4 == 0, "token rows per wave");
    constexpr uint32_t DAL = kqa ? 1 : 8 * TOK / (64 * NW);        // token-scale loads per wave
    constexpr uint32_t CPW = TPW / 4 + F::W16 + F::W4 + (k5 ? 0 : 1) + DAL + (has_qh(T) ? 1 : 0) + (mf ? 1 : has_m(T) ? DAL : 0) +
                             (k5 ? DBS : 0);
    // Weights: 16-byte piece P = 64*i + lane of the wave's area is row P/(RB/16), piece P%(RB/16);
    // rows of 256 or 128 bytes are swizzled (piece c of row r at c ^ (r & 15), resp. r & 7) so
    // the 32 rows one operand read covers hit distinct banks. Q6_K's 208-byte rows need no
    // swizzle; its last 512 bytes go as words.
    constexpr uint32_t PPR = F::RB / 16;
    uint32_t woff[F::W16 + F::W4];
#pragma unroll
    for (uint32_t i = 0; i < F::W16; i++) {
        const uint32_t P = 64 * i + lane, lr = P / PPR, pc = P % PPR;
        const uint32_t rr = clamp_row(r0 + 32 * wave + lr);
        const uint32_t c = unswz ? pc : (pc ^ (lr & (PPR - 1)));
        woff[i] = rr * nsb * F::RB + 16 * c;
    }
    if constexpr (unswz) {
#pragma unroll
        for (uint32_t i = 0; i < F::W4; i++) {
            const uint32_t Wd = 64 * 4 * F::W16 + 64 * i + lane; // 4-byte word of the wave's area
            const uint32_t rr = clamp_row(r0 + 32 * wave + Wd / (F::RB / 4));
            woff[F::W16 + i] = rr * nsb * F::RB + 4 * (Wd % (F::RB / 4));
        }
    }
    // Scales: Q6_K one f16 per row and step (the aligned dword holding it); the blocks' eight
    // f16 (16 bytes) per row and step otherwise. Lanes 32-63 repeat lanes 0-31.
    // Q4_0..Q5_1 (side plane per row: d[nbr], m[nbr], qh[nbr]): lanes 32-63 load m, and the
    // fifth-bit words of blocks 0-3 (lanes 0-31) and 4-7 (lanes 32-63) go as a second load.
    const uint32_t srow = clamp_row(r0 + 32 * wave + j);
    constexpr bool low4 = has_m(T) || has_qh(T) || zero_point(T) != 0;
    const SideGeom G = side_geom(T, K / 32);
    const uint32_t sidebase = srow * G.stride;
    const uint32_t sbase = q6 ? srow * nsb : !low4 ? srow * G.stride : sidebase + (h && has_m(T) ? G.m_off : 0);
    const uint32_t qhbase = sidebase + G.qh_off + 16 * h;
    const uint32_t xsoff = clamp_row(r0 + 32 * wave + lane / 2) * nsb * 8 + 4 * (lane % 2);
    // Q5_K d_a * bsum32: load i of wave m covers entries 64*(DBS*m + i) .. of [8][TOK]: sub-block
    // e / TOK, token e % TOK.
    uint32_t boff[k5 ? DBS : 1];
    if constexpr (k5) {
#pragma unroll
        for (uint32_t i = 0; i < DBS; i++) {
            const uint32_t e = 64 * (DBS * wave + i) + lane;
            boff[i] = clamp_tok(t0 + e % TOK) * (K / 32) * 4 + 4 * (e / TOK);
        }
    }
    // Token data: activation int8 rows, swizzled like the weights; token scales.
    uint32_t aoff[TPW / 4];
#pragma unroll
    for (uint32_t i = 0; i < TPW / 4; i++) {
        const uint32_t tl = TPW * wave + 4 * i + lane / 16;
        const uint32_t c = (lane % 16) ^ (tl & 15);
        aoff[i] = clamp_tok(t0 + tl) * K + 16 * c;
    }
    // Token scales: Q6_K lane L of wave m loads token 64m + L's; A8 load i of wave m covers the
    // 64 entries 64*(DAL*m + i) .. of the [8][TOK] array: block e / TOK, token e % TOK.
    uint32_t doff[DAL];
#pragma unroll
    for (uint32_t i = 0; i < DAL; i++) {
        if constexpr (kqa) {
            const uint32_t tl = 64 * wave + lane;
            doff[i] = clamp_tok(t0 + (tl < TOK ? tl : 0)) * nsb * 4;
        } else {
            const uint32_t e = 64 * (DAL * wave + i) + lane;
            doff[i] = clamp_tok(t0 + e % TOK) * (K / 32) * 4 + 4 * (e / TOK);
        }
    }

    // Q4_1 / Q5_1 offset operand: byte e = 1024*wave + 16*lane of the token range's 48-byte rows.
    constexpr uint32_t DSC = (TOK * 48 + 1023) / 1024; // 1-KB chunks of the offset operand
    static_assert(!mf || DSC <= NW, "one offset-operand load per wave");
    const uint32_t dsc = wave < DSC ? wave : DSC - 1;
    uint32_t dsboff = 0;
    if constexpr (mf) {
        const uint32_t e = 1024 * dsc + 16 * lane;
        dsboff = clamp_tok(t0 + e / 48) * 48 + e % 48;
    }
    auto issue = [&](uint32_t sb, Slot &S) {
        const int8_t *ga = a.aqs + 256 * sb;
#pragma unroll
        for (uint32_t i = 0; i < TPW / 4; i++) load_lds16(ga + aoff[i], &S.a[(TPW * wave + 4 * i) * 256]);
        const uint8_t *gw = a.w + uint64_t(sb) * F::RB;
#pragma unroll
        for (uint32_t i = 0; i < F::W16; i++) load_lds16(gw + woff[i], &S.w[wave][1024 * i]);
#pragma unroll
        for (uint32_t i = 0; i < F::W4; i++) load_lds4(gw + woff[F::W16 + i], &S.w[wave][1024 * F::W16 + 256 * i]);
        const uint8_t *gd = reinterpret_cast<const uint8_t *>(a.ad);
        if constexpr (q6) {
            load_lds4(a.ws + (((sbase + sb) >> 1) << 2), &S.ws[wave][0]);
            load_lds4(gd + doff[0] + 4 * sb, &S.da[64 * wave]);
        } else if constexpr (xs) {
            load_lds4(a.ws + xsoff + 8 * sb, &S.ws[wave][0]);
            load_lds4(gd + doff[0] + 4 * sb, &S.da[64 * wave]);
        } else if constexpr (k5) {
            load_lds4(gd + doff[0] + 4 * sb, &S.da[64 * wave]);
            const uint8_t *gb = reinterpret_cast<const uint8_t *>(a.adb);
#pragma unroll
            for (uint32_t i = 0; i < DBS; i++) load_lds4(gb + boff[i] + 32 * sb, &S.sa[64 * (DBS * wave + i)]);
        } else {
            load_lds16(a.ws + sbase + 16 * sb, &S.ws[wave][0]);
            if constexpr (has_qh(T)) load_lds16(a.ws + qhbase + 32 * sb, &S.ws[wave][1024]);
#pragma unroll
            for (uint32_t i = 0; i < DAL; i++) load_lds4(gd + doff[i] + 32 * sb, &S.da[64 * (DAL * wave + i)]);
            if constexpr (mf) {
                load_lds16(a.adsb + uint64_t(sb) * a.n * 48 + dsboff, &S.dsb[256 * dsc]);
            } else if constexpr (has_m(T)) {
                const uint8_t *gs = reinterpret_cast<const uint8_t *>(a.ads);
#pragma unroll
                for (uint32_t i = 0; i < DAL; i++) load_lds4(gs + doff[i] + 32 * sb, &S.sa[64 * (DAL * wave + i)]);
            }
        }
    };

    v16f acc[TT];
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.0f;

    // Step j of slice ks is super-block ks + KS*j (loads past the end repeat the last one).
    const uint32_t nst = (nsb + KS - 1) / KS;
    auto sb_of = [&](uint32_t st) {
        const uint32_t sb = ks + KS * st;
        return sb < nsb ? sb : nsb - 1;
    };
    issue(sb_of(0), slot_at(std::integral_constant<int, 0>{}));
    if constexpr (NB == 3) issue(sb_of(1), slot_at(std::integral_constant<int, 1>{}));
    __builtin_amdgcn_s_waitcnt((0x0F70 & ~0xF) | ((CPW * (NB - 2)) & 0xF) | (((CPW * (NB - 2)) >> 4) << 14));
    __syncthreads();

    const uint32_t sw = j & 15;
    auto step = [&](auto ic, uint32_t st) {
        constexpr int I = decltype(ic)::value;
        issue(sb_of(st + NB - 1), slot_at(std::integral_constant<int, (I + NB - 1) % NB>{}));
        Slot &S = slot_at(ic);
        const uint32_t sb = ks + KS * st;
        if (KS > 1 && sb >= nsb) {
            __builtin_amdgcn_s_waitcnt((0x0F70 & ~0xF) | ((CPW * (NB - 2)) & 0xF) | (((CPW * (NB - 2)) >> 4) << 14));
            __syncthreads();
            return;
        }
        const int8_t *abase = &S.a[j * 256];
        v4i av[8];
        auto load_a = [&](int t) {
#pragma unroll
            for (int c = 0; c < 8; c++)
                av[c] = *reinterpret_cast<const v4i *>(abase + 32 * t * 256 + 16 * ((2 * c + h) ^ sw));
        };

        if constexpr (q6) {
            // This lane's row half: group 2c + h of chunk c = 4n + p is ql bytes 64n + 32(p&1) +
            // 16h.. (nibble p>>1), qh bytes 128 + 32n + 16h.. (bits 2p), scale byte 192 + 8n + 2p + h
            // (dequant.zig's Q6_K order).
            const uint8_t *blk = &S.w[wave][208 * j];
            uint4 ql[2][2], qh[2];
#pragma unroll
            for (int n = 0; n < 2; n++) {
#pragma unroll
                for (int pp = 0; pp < 2; pp++) ql[n][pp] = *reinterpret_cast<const uint4 *>(blk + 64 * n + 32 * pp + 16 * h);
                qh[n] = *reinterpret_cast<const uint4 *>(blk + 128 + 32 * n + 16 * h);
            }
            const uint4 scw = *reinterpret_cast<const uint4 *>(blk + 192);
            const uint32_t scs[4] = {scw.x, scw.y, scw.z, scw.w};
            const uint32_t dword = *reinterpret_cast<const uint32_t *>(&S.ws[wave][4 * j]);
            const float d = f16_bits_to_f32(((sbase + sb) & 1) ? dword >> 16 : dword & 0xFFFF);
            // Planes H, L of the group-scaled weights (4*w = 256*H + L).
            v4i P[2][8];
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int n = c / 4, p = c % 4;
                const uint32_t sbyte = 8 * n + 2 * p + h;
                const int sc = int(int8_t((scs[sbyte / 4] >> (8 * (sbyte % 4))) & 0xFF));
                const uint32_t m = q6k_m(sc), k = q6k_k(sc);
                const uint32_t qlw[4] = {ql[n][p & 1].x, ql[n][p & 1].y, ql[n][p & 1].z, ql[n][p & 1].w};
                const uint32_t qhw[4] = {qh[n].x, qh[n].y, qh[n].z, qh[n].w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t q = ((qlw[i] >> (4 * (p >> 1))) & 0x0F0F0F0Fu) | (((qhw[i] >> (2 * p)) & 0x03030303u) << 4);
                    int hp, lp;
                    q6k_planes(q, m, k, hp, lp);
                    P[0][c][i] = hp;
                    P[1][c][i] = lp;
                }
            }
            const float d4 = 0.25f * d;
            load_a(0);
#pragma unroll
            for (int t = 0; t < TT; t++) {
                v16i sacc = {};
#pragma unroll
                for (int c = 0; c < 8; c++) sacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[c], P[0][c], sacc, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; v++) sacc[v] <<= 8;
#pragma unroll
                for (int c = 0; c < 8; c++) sacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[c], P[1][c], sacc, 0, 0, 0);
                if (t + 1 < TT) load_a(t + 1);
                const float4 *dap = reinterpret_cast<const float4 *>(&S.da[32 * t + 4 * h]);
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const float4 dv = dap[2 * g];
                    const float ds[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[t][4 * g + e] = fmaf((float)sacc[4 * g + e], d4 * ds[e], acc[t][4 * g + e]);
                }
            }
        } else {
            // Block c of this lane's row: its 16-byte piece (Q8_0: bytes 16h.. of the block;
            // IQ4_NL: the block's 16 bytes, low nibbles for h = 0, high for h = 1).
            const uint8_t *blk = &S.w[wave][F::RB * j];
            v4i wv[8];
            float dw[8], mw[8];
            if constexpr (k5) {
                // Sub-block c of this lane's row half: nibble c%2 of qs bytes 32(c/2) + 16h.., fifth
                // bit c of qh bytes 16h.. (k4Block has_high); scales and mins by the word unpack
                // (vecdot.zig:461-474).
                const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
                const uint4 qh4 = *reinterpret_cast<const uint4 *>(blk + 16 + 16 * h);
                const uint32_t qhw[4] = {qh4.x, qh4.y, qh4.z, qh4.w};
                const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
                const uint32_t scw[2] = {hd.y & k1, (hd.w & k2) | (((hd.y >> 6) & k3) << 4)};
                const uint32_t mnw[2] = {hd.z & k1, ((hd.w >> 4) & k2) | (((hd.z >> 6) & k3) << 4)};
                const float d = f16_bits_to_f32(hd.x & 0xFFFF), dmin = f16_bits_to_f32(hd.x >> 16);
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const uint4 x = *reinterpret_cast<const uint4 *>(blk + 48 + 32 * (c / 2) + 16 * h);
                    const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        wv[c][i] = int(((xw[i] >> (4 * (c & 1))) & 0x0F0F0F0Fu) | (((qhw[i] >> c) & 0x01010101u) << 4));
                    dw[c] = d * (float)((scw[c / 4] >> (8 * (c % 4))) & 0xFF);
                    mw[c] = dmin * (float)((mnw[c / 4] >> (8 * (c % 4))) & 0xFF);
                }
            }
#pragma unroll
            for (int c = 0; c < 8; c++) {
                if constexpr (k5) {
                } else if constexpr (T == HKHIP_Q8_0) {
                    wv[c] = *reinterpret_cast<const v4i *>(blk + 16 * ((2 * c + h) ^ sw));
                } else {
                    const uint4 x = *reinterpret_cast<const uint4 *>(blk + 16 * (c ^ (j & 7)));
                    const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
                    uint32_t qh = 0;
                    constexpr int TL = xs ? HKHIP_IQ4_NL : T; // IQ4_XS: IQ4_NL's codebook
                    if constexpr (has_qh(T))
                        qh = *reinterpret_cast<const uint32_t *>(&S.ws[wave][1024 + 16 * (32 * (c / 4) + j) + 4 * (c % 4)]);
#pragma unroll
                    for (int i = 0; i < 4; i++) wv[c][i] = int(low_bit_word<TL>(xw[i], qh, h, i));
                }
            }
            // Q4_1 / Q5_1 offset term, sum_c m[r,c] * (d_a * s)[t,c] over the super-block's 8 blocks,
            // on bf16 MFMAs: m (an f16) is hi + lo exactly (8 + at most 3 significant bits), the
            // token side hi + mid + lo (a8_dsb); three 32x32x16 MFMAs pair (hi|mid) with m's hi and
            // lo and the token lo with m's hi -- every partial product down to 2^-24 relative.
            v8bf mB1, mB2, mB3;
            if constexpr (has_m(T) && !mf) {
                const uint4 m16 = *reinterpret_cast<const uint4 *>(&S.ws[wave][16 * (32 + j)]);
                const uint32_t mw4[4] = {m16.x, m16.y, m16.z, m16.w};
#pragma unroll
                for (int c = 0; c < 8; c++) mw[c] = f16_bits_to_f32((mw4[c / 2] >> (16 * (c & 1))) & 0xFFFF);
            } else if constexpr (mf) {
                const uint4 m16 = *reinterpret_cast<const uint4 *>(&S.ws[wave][16 * (32 + j)]);
                const uint32_t mw4[4] = {m16.x, m16.y, m16.z, m16.w};
                uint32_t mh[4], ml[4];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    uint32_t hi2[2], lo2[2];
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const float m = f16_bits_to_f32((mw4[q] >> (16 * e)) & 0xFFFF);
                        hi2[e] = __builtin_bit_cast(uint32_t, m) & 0xFFFF0000u;
                        lo2[e] = __builtin_bit_cast(uint32_t, m - __builtin_bit_cast(float, hi2[e]));
                    }
                    mh[q] = __builtin_amdgcn_perm(hi2[1], hi2[0], 0x07060302u);
                    ml[q] = __builtin_amdgcn_perm(lo2[1], lo2[0], 0x07060302u);
                }
                mB1 = __builtin_bit_cast(v8bf, make_uint4(mh[0], mh[1], mh[2], mh[3]));
                mB2 = __builtin_bit_cast(v8bf, make_uint4(ml[0], ml[1], ml[2], ml[3]));
                mB3 = h ? v8bf{} : mB1;
            }
            if constexpr (k5) {
            } else if constexpr (xs) {
                // d * ls_c (exact in f32): ls_c = scales_l nibble | scales_h bits << 4, minus 32
                // (dequant.zig:443-447).
                const uint2 hd = *reinterpret_cast<const uint2 *>(&S.ws[wave][8 * j]);
                const float d = f16_bits_to_f32(hd.x & 0xFFFF);
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const uint32_t lo = (hd.y >> (4 * c)) & 0xF, hi = (hd.x >> (16 + 2 * c)) & 3;
                    dw[c] = d * (float)(int(lo | (hi << 4)) - 32);
                }
            } else {
                const uint4 s16 = *reinterpret_cast<const uint4 *>(&S.ws[wave][16 * j]);
                const uint32_t sw4[4] = {s16.x, s16.y, s16.z, s16.w};
#pragma unroll
                for (int c = 0; c < 8; c++) dw[c] = f16_bits_to_f32((sw4[c / 2] >> (16 * (c & 1))) & 0xFFFF);
            }
            load_a(0);
#pragma unroll
            for (int t = 0; t < TT; t++) {
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const v16i p = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[c], wv[c], v16i{}, 0, 0, 0);
                    // Scales of this lane's 16 outputs: tokens 32t + 8g + 4h + (0..3).
                    const float4 *dap = reinterpret_cast<const float4 *>(&S.da[(xs || k5 ? 0 : c * TOK) + 32 * t + 4 * h]);
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const float4 dv = dap[2 * g];
                        const float ds[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            acc[t][4 * g + e] = fmaf((float)p[4 * g + e], dw[c] * ds[e], acc[t][4 * g + e]);
                        if constexpr (has_m(T) && !mf) {
                            const float4 sv = *reinterpret_cast<const float4 *>(&S.sa[c * TOK + 32 * t + 4 * h + 8 * g]);
                            const float dss[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
                            for (int e = 0; e < 4; e++) acc[t][4 * g + e] = fmaf(mw[c], dss[e], acc[t][4 * g + e]);
                        }
                        if constexpr (k5) { // - dmin * mn_c * (da * bsum32_c)
                            const float4 bv = *reinterpret_cast<const float4 *>(&S.sa[c * TOK + 32 * t + 4 * h + 8 * g]);
                            const float db[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
                            for (int e = 0; e < 4; e++) acc[t][4 * g + e] = fmaf(-mw[c], db[e], acc[t][4 * g + e]);
                        }
                    }
                }
                if constexpr (mf) {
                    const uint32_t *tm = &S.dsb[12 * (32 * t + j)];
                    const v8bf a12 = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4 *>(tm + 4 * h));
                    const v8bf a3 = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4 *>(tm + 8));
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a12, mB1, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a12, mB2, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a3, mB3, acc[t], 0, 0, 0);
                }
                if (t + 1 < TT) load_a(t + 1);
            }
        }
        __builtin_amdgcn_s_waitcnt((0x0F70 & ~0xF) | ((CPW * (NB - 2)) & 0xF) | (((CPW * (NB - 2)) >> 4) << 14));
        __syncthreads();
    };
    for (uint32_t st = 0; st < nst; st += NB) {
        step(std::integral_constant<int, 0>{}, st);
        if (st + 1 < nst) step(std::integral_constant<int, 1>{}, st + 1);
        if constexpr (NB == 3)
            if (st + 2 < nst) step(std::integral_constant<int, 2>{}, st + 2);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): no direct load still writing the ring
    __syncthreads();                   // in any wave: the ring is free from here

    if constexpr (KS > 1) {
        // Slices 1.. leave their tiles in the ring; slice 0 adds them in order.
        float *red = reinterpret_cast<float *>(&ring0[0]);
        static_assert((KS - 1) * NW * TT * 16 * 64 * 4 <= KS * sizeof(Slot), "reduction space");
        if (ks > 0) {
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int v = 0; v < 16; v++) red[((((ks - 1) * NW + wave) * TT + t) * 16 + v) * 64 + lane] = acc[t][v];
        }
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int k = 1; k < KS; k++)
#pragma unroll
                for (int t = 0; t < TT; t++)
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[t][v] += red[((((k - 1) * NW + wave) * TT + t) * 16 + v) * 64 + lane];
        }
        __syncthreads(); // the reduction area is read: the ring takes the output staging
        if (ks > 0) return;
    }

    // ---- store: y[token][row], bias, accumulate ----
    {
        static_assert(NW * 4096 <= KS * sizeof(Slot), "output staging space");
        float *st = reinterpret_cast<float *>(&ring0[0]) + 1024 * wave;
        const float b = (a.bias && myrow < a.rows) ? a.bias[myrow] : 0.0f;
        const uint32_t rw0 = r0 + 32 * wave;
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const uint32_t tk0 = t0 + 32 * t;
            if (a.wide && rw0 + 32 <= a.rows && tk0 + 32 <= a.n)
                gemm_store_tile_wide(st, acc[t], b, a.y, a.rows, rw0, tk0, a.mode);
            else
                gemm_store_tile(acc[t], b, a.y, a.rows, a.n, myrow, tk0, a.mode);
        }
    }
}

typedef void (*mx_kernel_t)(MxArgs);

template <int T, int NW, int TT, int NB, int KS = 1>
hipError_t launch_cfg(const MxArgs &a0, hipStream_t s) {
    static_assert(NB * KS * sizeof(MxSlot<T, 32 * TT, NW, KS == 1>) <= 160 * 1024, "LDS");
    MxArgs a = a0;
    a.rblocks = (a.rows + 32 * NW - 1) / (32 * NW);
    a.tblocks = (a.n + 32 * TT - 1) / (32 * TT);
    hipLaunchKernelGGL((mmx_kernel<T, NW, TT, NB, KS>), dim3(a.rblocks * a.tblocks), dim3(NW * KS * 64), 0, s, a);
    return hipGetLastError();
}

// Q4_0..Q5_1: IQ4_NL's tile choice (same quant bytes per block).
template <int T> hipError_t launch_low4(const MxArgs &a, hipStream_t s, uint32_t b82, uint32_t b42) {
    if (b82 >= 224) return launch_cfg<T, 8, 2, 2>(a, s);
    if constexpr (has_qh(T)) { // two K slices would not fit the LDS with the fifth-bit words
        if (b42 >= 128) return launch_cfg<T, 4, 2, 2>(a, s);
    } else {
        if (b42 >= 128 && a.cols >= 1024) return launch_cfg<T, 4, 2, 2, 2>(a, s);
    }
    // Long rows and few row blocks or tokens (measured at the 8B FFN shapes, 9-64 tokens): 64-row
    // tiles split over K slices (Q4_1 4096 x 14336: 127 -> 50 us, 14336 x 4096 at <= 32 tokens:
    // 40 -> 19 us). Not for Q4_0, which measured slower so (104 -> 120 us), nor for 14336 rows
    // past one token tile (the grid doubles: 34 -> 74 us).
    if (T != HKHIP_Q4_0 && a.cols >= 4096 && (a.rows < 8192 || a.n <= 32)) {
        if constexpr (has_qh(T))
            return launch_cfg<T, 2, 1, 2, 2>(a, s);
        else
            return launch_cfg<T, 2, 1, 2, 4>(a, s);
    }
    return launch_cfg<T, 4, 1, 2>(a, s);
}

} // namespace mx

bool mmx_supports(int t, uint32_t rows, uint32_t cols, uint32_t n) {
    if (t != HKHIP_Q6_K && t != HKHIP_IQ4_XS && t != HKHIP_Q5_K && !legacy32(t)) return false;
    if (cols % 256 != 0 || rows == 0 || n == 0) return false;
    // 32-bit per-lane byte offsets: quant plane, scale plane and activations.
    const WLayout W = weight_layout(t, rows, cols);
    return W.total < (1ull << 32) && uint64_t(n) * cols < (1ull << 32);
}

hipError_t launch_mmx(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n, float *y,
                      const float *bias, int mode, hipStream_t s) {
    if (!mmx_supports(t, rows, cols, n)) return hipErrorInvalidValue;
    const WLayout W = weight_layout(t, rows, cols);
    const ActLayout A = act_layout(n, cols);
    const bool q6 = act_kind(t) == HKHIP_ACT_Q8K; // Q6_K, IQ4_XS
    mx::MxArgs a{};
    a.w = w;
    a.ws = w + W.scale_off;
    a.rows = rows;
    a.cols = cols;
    a.n = n;
    a.aqs = reinterpret_cast<const int8_t *>(xq + (q6 ? A.k_qs : A.a8_qs));
    a.ad = reinterpret_cast<const float *>(xq + (q6 ? A.k_d : A.a8_d));
    a.ads = reinterpret_cast<const float *>(xq + A.a8_ds);
    a.adsb = xq + A.a8_dsb;
    a.adb = reinterpret_cast<const float *>(xq + A.k_db);
    a.y = y;
    a.bias = bias;
    a.mode = mode;
    a.wide = (reinterpret_cast<uintptr_t>(y) % 16 == 0 && rows % (mode == HKHIP_SILU_MUL ? 8 : 4) == 0) ? 1 : 0;
    // Tile choice (measured at the 8B FFN shapes, 512 tokens): the largest tile that still gives
    // most CUs a workgroup.
    auto blocks = [&](uint32_t nw, uint32_t tt) {
        return ((rows + 32 * nw - 1) / (32 * nw)) * ((n + 32 * tt - 1) / (32 * tt));
    };
    switch (t) {
    case HKHIP_Q6_K:
        if (blocks(4, 2) >= 192) return mx::launch_cfg<HKHIP_Q6_K, 4, 2, 2>(a, s);
        return mx::launch_cfg<HKHIP_Q6_K, 4, 1, 2>(a, s);
    case HKHIP_Q8_0:
        return mx::launch_cfg<HKHIP_Q8_0, 4, 1, 2>(a, s);
    case HKHIP_IQ4_NL:
        // Few row blocks (4096 x 14336: 139 vs 234 us): two K slices instead of 256-row tiles.
        if (blocks(8, 2) >= 224) return mx::launch_cfg<HKHIP_IQ4_NL, 8, 2, 2>(a, s);
        if (blocks(4, 2) >= 128 && cols >= 1024) return mx::launch_cfg<HKHIP_IQ4_NL, 4, 2, 2, 2>(a, s);
        return mx::launch_cfg<HKHIP_IQ4_NL, 4, 1, 2>(a, s);
    case HKHIP_Q4_0: return mx::launch_low4<HKHIP_Q4_0>(a, s, blocks(8, 2), blocks(4, 2));
    case HKHIP_Q4_1: return mx::launch_low4<HKHIP_Q4_1>(a, s, blocks(8, 2), blocks(4, 2));
    case HKHIP_Q5_0: return mx::launch_low4<HKHIP_Q5_0>(a, s, blocks(8, 2), blocks(4, 2));
    case HKHIP_Q5_1: return mx::launch_low4<HKHIP_Q5_1>(a, s, blocks(8, 2), blocks(4, 2));
    case HKHIP_Q5_K: // the offset term makes it Q4_1-like; two K slices do not fit with 176-B rows
        if (blocks(4, 2) >= 160) return mx::launch_cfg<HKHIP_Q5_K, 4, 2, 2>(a, s);
        return mx::launch_cfg<HKHIP_Q5_K, 4, 1, 2>(a, s);
    case HKHIP_IQ4_XS:
        if (blocks(8, 2) >= 224) return mx::launch_cfg<HKHIP_IQ4_XS, 8, 2, 2>(a, s);
        if (blocks(4, 2) >= 128 && cols >= 1024) return mx::launch_cfg<HKHIP_IQ4_XS, 4, 2, 2, 2>(a, s);
        if (cols >= 4096 && (rows < 8192 || n <= 32)) return mx::launch_cfg<HKHIP_IQ4_XS, 2, 1, 2, 4>(a, s);
        return mx::launch_cfg<HKHIP_IQ4_XS, 4, 1, 2>(a, s);
    default: return hipErrorInvalidValue;
    }
}

} // namespace hkhip
