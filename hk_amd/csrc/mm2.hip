// Prefill GEMM for Q4_K on the int8 MFMA units, split-plane form.
//
// Per row r, token t and super-block b, hk's CPU kernel (src/quant/gemm.zig kernelK 180-236,
// with the scale unpack of unpack.zig) computes
//     y[t][r] += d[r,b]*da[t,b] * sum_s sc[r,b,s] * sum_{k in s} q[r,k]*a[t,k]
//              - dmin[r,b]*da[t,b] * sum_s mn[r,b,s] * bsum32[t,b,s]
// with exact integer inner sums. Here:
//  * main term: the 6-bit sub-block scale is folded into the weights as two int8 planes: with
//    sc = 8*sh + sl (sh, sl in [0,7]), sc*q = 8*(sh*q) + (sl*q) and both products are at most
//    105, so one packed 16-bit multiply makes a plane for four weights without carries between
//    bytes. Two int32 MFMA chains over the super-block's 256 weights give sum(sh*q*a) and
//    sum(sl*q*a), combined exactly as (h << 3) + l -- the same integer as the reference's -- and
//    applied with one f32 update per super-block.
//  * min term: J = sum_s mn[s]*bsum32[s] is an integer below 2^22, and both factors are exact
//    bf16 integers once bsum32 is written as 64*u + v (v in [0, 63]). The staged kernels run one
//    32x32x16 bf16 MFMA with 64*u in its first 8 k and v in the other 8 (against mn in both),
//    which yields J exactly in f32, and apply both terms in one update: y += da*(d*I - dmin*J).
//    The large-tile kernel has no registers left for J's tile, so it folds the float scales into
//    the operands instead, (-dmin*mn) x (da*bsum32), each split into three bf16 parts (their sum
//    is the fp32 value to within 2^-24): a 32x32x16 MFMA pairs 8 sub-blocks of one token part
//    (first 8 k) and another (last 8 k) with a row part, so three of them, (hi|mid) x h,
//    (hi|mid) x m, (hi|lo) x (l|h), form every partial product down to 2^-24, accumulated in f32
//    straight into the output tile.
// Only the f32 summation order differs from the reference.
//
// Tiling: a workgroup of 8 waves (two per SIMD, so one wave's VALU work and LDS waits overlap
// the other's MFMAs) owns 256 rows x 128 tokens; a wave owns 32 rows (its lanes' rows, so a
// row's scales are per-lane scalars) x 128 tokens (4 MFMA tiles of 32x32). Weights are private
// to a wave: each lane loads and unpacks its row's half of every super-block straight from HBM
// into MFMA operand registers. Activations are shared: the workgroup stages each super-block's
// 128 tokens x 256 int8 (+ the scales and the min-term operand) in LDS, double buffered, one
// barrier per super-block.
//
// MFMA roles: A = activations (tokens as M), B = weights (rows as N). Output lane l holds row
// l%32 and tokens 8*(v/4) + 4*(l/32) + v%4 for v < 16.

#include "common.hpp"
#include "gemm_store.hpp"

#include <type_traits>

namespace hkhip {


typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef short s2v __attribute__((ext_vector_type(2)));

// Shapes: NW waves per workgroup (32 rows each), TT token tiles of 32 per wave, NB super-blocks
// in flight; the workgroup covers 32*NW rows x 32*TT tokens. The large configuration amortizes
// the weight unpack over 128 tokens; smaller ones keep small matrices spread over the CUs.
// Everything a super-block needs arrives by direct global -> LDS loads into a ring of NB slots:
//   a   token rows, 256 int8 each; 16-byte chunk c of token t sits at c ^ (t & 15) so the 32
//       tokens one MFMA operand read covers hit distinct banks
//   w   per wave, its 32 rows' 144-byte blocks back to back
//   mb  per token, the min-term operand (k_mb of the activation buffer, 32 bytes)
//   da  per token, the Q8K scale
// Every wave issues the same loads (waves past the tokens load duplicates into their own spare
// entries), so the in-order memory counter can be waited on with a constant.
template <int TOK, int NW, int WB = 4608> struct Q2Slot {
    int8_t a[TOK * 256];
    uint8_t w[NW][WB]; // 32 rows x 144 (Q4_K) or 176 (Q5_K) bytes
    uint32_t mb[NW * 32][8]; // token t at mb[t]; wave m's load fills tokens 32m..32m+31
    float da[NW * 64];       // token t at da[t]; wave m's load fills tokens 64m..64m+63
};

struct Mm2Args {
    const uint8_t *w;
    uint32_t rows, cols, n;
    const int8_t *aqs;
    const float *ad;
    const int16_t *abs;
    const uint8_t *amb; // k_mb: per token and super-block, 32 bytes (64*u, then v, as bf16)
    float *y;
    const float *bias;
    int mode;
    int wide; // y 16-byte aligned and rows a multiple of 4: whole tiles go out as 16-byte stores
    uint32_t rblocks, tblocks;
};

__device__ __forceinline__ uint4 ldg16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }

// x as three bf16 parts hi + mid + lo, each the top 16 bits of an f32 (the low 16 bits of the
// returned words are left as they fall): hi keeps x's leading 8 significant bits, mid the next 8
// of the remainder, lo the rest, which then has at most 8 -- so the sum is x exactly.
__device__ __forceinline__ void bf16_split3(float x, uint32_t p[3]) {
    p[0] = __builtin_bit_cast(uint32_t, x) & 0xFFFF0000u;
    const float r1 = x - __builtin_bit_cast(float, p[0]);
    p[1] = __builtin_bit_cast(uint32_t, r1) & 0xFFFF0000u;
    p[2] = __builtin_bit_cast(uint32_t, r1 - __builtin_bit_cast(float, p[1]));
}
// Two split values as bf16 pairs, x0 in the low half: the top halves of a and b.
__device__ __forceinline__ uint32_t bf16_pair(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// Row-side min-term operands of one super-block: -dmin*mn of the 8 sub-blocks (6-bit mins in
// the bytes of mnl, mnh) in three bf16 parts, as the B operands of the three 32x32x16 MFMAs:
// hi and mid in both lane halves, then lo in half 0 and hi in half 1.
struct MinB {
    v8bf b1, b2, b3;
};
__device__ __forceinline__ MinB min_operands(uint32_t mnl, uint32_t mnh, float dmin, uint32_t h) {
    uint32_t w[3][4];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        uint32_t p[3];
        bf16_split3(-dmin * (float)(((s < 4 ? mnl : mnh) >> (8 * (s & 3))) & 0xFF), p);
#pragma unroll
        for (int q = 0; q < 3; q++) {
            if (s & 1)
                w[q][s / 2] = bf16_pair(w[q][s / 2], p[q]);
            else
                w[q][s / 2] = p[q];
        }
    }
    MinB m;
    m.b1 = __builtin_bit_cast(v8bf, make_uint4(w[0][0], w[0][1], w[0][2], w[0][3]));
    m.b2 = __builtin_bit_cast(v8bf, make_uint4(w[1][0], w[1][1], w[1][2], w[1][3]));
    const uint32_t q = h ? 0 : 2;
    m.b3 = __builtin_bit_cast(v8bf, make_uint4(w[q][0], w[q][1], w[q][2], w[q][3]));
    return m;
}

// Adds the min term of one 32x32 tile: tm = the 12 words (hi, mid, lo: 8 bf16 each) of this
// lane's token, B = the row side.
__device__ __forceinline__ void min_term(v16f &acc, const uint32_t *tm, const MinB &B, uint32_t h) {
    const v8bf a12 = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4 *>(tm + 4 * h)); // hi | mid
    const v8bf a3 = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4 *>(tm + 8 * h));  // hi | lo
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a12, B.b1, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a12, B.b2, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a3, B.b3, acc, 0, 0, 0);
}

// Row-side operand of the min term: the 8 sub-blocks' 6-bit mins (bytes of mnl, mnh) as bf16
// integers, the same 8 values in both lane halves.
__device__ __forceinline__ v8bf min_b(uint32_t mnl, uint32_t mnh) {
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t src = q < 2 ? mnl : mnh, sh = 16 * (q & 1);
        const float e = (float)((src >> sh) & 0xFF), o = (float)((src >> (sh + 8)) & 0xFF);
        w[q] = (__builtin_bit_cast(uint32_t, e) >> 16) | (__builtin_bit_cast(uint32_t, o) & 0xFFFF0000u);
    }
    return __builtin_bit_cast(v8bf, make_uint4(w[0], w[1], w[2], w[3]));
}

// J = sum_s mn[s] * bsum32[s] of a 32x32 tile, exact: tm holds this lane's token's 8 words
// (64*u of the 8 sub-blocks in words 0-3, v in 4-7); lane half h supplies its half. `after` is
// a value the caller computes just before: the operand is tied to it so that the MFMA is not
// hoisted (with its result registers) ahead of the tile's other work.
__device__ __forceinline__ v16f min_j(const uint32_t *tm, v8bf mn, uint32_t h, float after) {
    uint4 w = *reinterpret_cast<const uint4 *>(tm + 4 * h);
    asm volatile("" : "+v"(w.x) : "v"(after));
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, w), mn, v16f{}, 0, 0, 0);
}

// Q5_K: four 5-bit quants u (bytes; even bytes ev, odd od, as 16-bit lanes) times a factor e
// in [0, 7], minus 16e: per byte (u - 16)*e in [-112, 105] as a two's-complement byte (packed
// 16-bit multiply-adds keep the bytes apart; the low byte of each lane is the wanted one).
// -16e in both 16-bit lanes, for a factor e held as e * 0x00010001.
__device__ __forceinline__ uint32_t neg16(uint32_t m) { return ((0u - 16u * (m & 0xFFFFu)) & 0xFFFFu) * 0x00010001u; }
__device__ __forceinline__ uint32_t plane_c16(uint32_t ev, uint32_t od, uint32_t m, uint32_t c) {
    const us2 pe = __builtin_bit_cast(us2, ev) * __builtin_bit_cast(us2, m) + __builtin_bit_cast(us2, c);
    const us2 po = __builtin_bit_cast(us2, od) * __builtin_bit_cast(us2, m) + __builtin_bit_cast(us2, c);
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, po), __builtin_bit_cast(uint32_t, pe), 0x06020400u);
}

// Q5_K's row-side min-term operand: per sub-block s, 16*d*sc_s - dmin*mn_s (the weights enter
// the planes as u - 16, and 16*sum(sc*a) = 16*sc*bsum32 returns through the min term), split as
// min_operands does.
__device__ __forceinline__ MinB min_operands_k5(uint32_t scl, uint32_t sch, float d, uint32_t mnl, uint32_t mnh,
                                                float dmin, uint32_t h) {
    uint32_t w[3][4];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        uint32_t p[3];
        const float sc = (float)(((s < 4 ? scl : sch) >> (8 * (s & 3))) & 0xFF);
        const float mn = (float)(((s < 4 ? mnl : mnh) >> (8 * (s & 3))) & 0xFF);
        bf16_split3(16.0f * d * sc - dmin * mn, p);
#pragma unroll
        for (int q = 0; q < 3; q++) {
            if (s & 1)
                w[q][s / 2] = bf16_pair(w[q][s / 2], p[q]);
            else
                w[q][s / 2] = p[q];
        }
    }
    MinB m;
    m.b1 = __builtin_bit_cast(v8bf, make_uint4(w[0][0], w[0][1], w[0][2], w[0][3]));
    m.b2 = __builtin_bit_cast(v8bf, make_uint4(w[1][0], w[1][1], w[1][2], w[1][3]));
    const uint32_t q = h ? 0 : 2;
    m.b3 = __builtin_bit_cast(v8bf, make_uint4(w[q][0], w[q][1], w[q][2], w[q][3]));
    return m;
}

// Four nibble bytes (values 0..15) times a 3-bit scale factor: each byte product is at most
// 105, so a packed 16-bit multiply of the word keeps every byte separate.
__device__ __forceinline__ uint32_t mul_bytes(uint32_t nib, uint32_t f2) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(us2, nib) * __builtin_bit_cast(us2, f2));
}

template <int TOK, int NW> struct Q2Smem {
    int8_t a[2][TOK * 256];
    uint32_t mb[2][TOK][12]; // per token: 8 bf16 hi (words 0-3), mid (4-7), lo (8-11)
    float da[2][TOK];
    float st[NW][1024]; // per wave: a 32x32 output tile transposed for its stores
};

// Large-tile variant: weights go global -> registers (each lane its own row half), loaded
// while the previous super-block computes; activations and token data through LDS, double
// buffered. Measured faster than staging the weights in LDS for this tile.
// Q5_K (T = HKHIP_Q5_K) runs the same tile: the fifth bits come from the lane's half of qh, the
// planes hold (u - 16)*sh and (u - 16)*sl, and the min term carries 16*d*sc - dmin*mn.
template <int T, int Q2_NW, int Q2_TT>
__global__ __launch_bounds__(Q2_NW * 64, 2) void mm2_q4k_reg_kernel(Mm2Args a) {
    constexpr int Q2_ROWS = 32 * Q2_NW, Q2_TOK = 32 * Q2_TT;
    constexpr bool k5 = (T == HKHIP_Q5_K);
    constexpr uint32_t BB = k5 ? 176 : 144, QO = k5 ? 48 : 16; // block bytes, qs offset
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
    Q2Smem<Q2_TOK, Q2_NW> &S = *reinterpret_cast<Q2Smem<Q2_TOK, Q2_NW> *>(smem_raw);
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t h = lane >> 5, j = lane & 31;
    const uint32_t K = a.cols, nsb = K / 256;

    // Workgroup -> (row block, token block). The token blocks of one row block are consecutive
    // workgroups on the same XCD (workgroups go round-robin over the 8 XCDs), so the rows they
    // share are read from HBM once and then served by that XCD's L2.
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
    const uint32_t r0 = rb * Q2_ROWS, t0 = tb * Q2_TOK;
    const uint32_t myrow = r0 + 32 * wave + j;
    const uint32_t wrow = myrow < a.rows ? myrow : a.rows - 1;
    const uint8_t *wbase = a.w + uint64_t(wrow) * nsb * BB;

    // ---- staging of one super-block of activations ----
    // The int8 values go global -> LDS directly (global_load_lds_dwordx4: lane L of a wave writes
    // 16 bytes at the wave's LDS pointer + 16*L), 4 x 1 KB per wave = 16 token rows; the
    // swizzle is applied on the global side. Threads below 128 load token tid's scale and bsums
    // into registers and write the min-term operand after the compute.
    float sda = 0.0f;
    uint4 sbs0 = make_uint4(0, 0, 0, 0), sbs1 = sbs0;
    const bool tok_thread = tid < Q2_TOK;
    auto stage_load = [&](uint32_t sb, uint32_t buf) {
        // Each wave moves TPW token rows, 4 per 1-KB direct load.
        constexpr uint32_t TPW = Q2_TOK / Q2_NW;
        static_assert(TPW % 4 == 0, "token rows per wave");
#pragma unroll
        for (uint32_t i = 0; i < TPW / 4; i++) {
            const uint32_t tl = TPW * wave + 4 * i + lane / 16; // token row in the workgroup
            const uint32_t c = (lane % 16) ^ (tl & 15);         // chunk this lane's 16 bytes hold
            const uint32_t tok = t0 + tl, tk = tok < a.n ? tok : a.n - 1;
            load_lds16(a.aqs + uint64_t(tk) * K + 256 * sb + 16 * c, &S.a[buf][(TPW * wave + 4 * i) * 256]);
        }
        if (tok_thread) {
            const uint32_t tok = t0 + tid, tk = tok < a.n ? tok : a.n - 1;
            sda = a.ad[uint64_t(tk) * nsb + sb];
            const int16_t *bs = a.abs + uint64_t(tk) * (K / 16) + 16 * sb;
            sbs0 = ldg16(bs);
            sbs1 = ldg16(bs + 8);
        }
    };
    auto stage_store = [&](uint32_t buf) {
        if (tok_thread) {
            const bool ok = t0 + tid < a.n;
            const uint32_t bw[8] = {sbs0.x, sbs0.y, sbs0.z, sbs0.w, sbs1.x, sbs1.y, sbs1.z, sbs1.w};
            uint32_t w[3][4];
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const int b32 = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2v, bw[s]), s2v{1, 1}, 0, false);
                uint32_t p[3];
                bf16_split3(ok ? sda * (float)b32 : 0.0f, p);
#pragma unroll
                for (int q = 0; q < 3; q++) {
                    if (s & 1)
                        w[q][s / 2] = bf16_pair(w[q][s / 2], p[q]);
                    else
                        w[q][s / 2] = p[q];
                }
            }
            uint4 *mb = reinterpret_cast<uint4 *>(S.mb[buf][tid]);
#pragma unroll
            for (int q = 0; q < 3; q++) mb[q] = make_uint4(w[q][0], w[q][1], w[q][2], w[q][3]);
            S.da[buf][tid] = ok ? sda : 0.0f;
        }
    };

    // ---- this lane's weights: its row's half (h) of a super-block ----
    uint4 wh, wq[4], wx;
    auto wload = [&](uint32_t sb) {
        const uint8_t *blk = wbase + uint64_t(sb) * BB;
        wh = ldg16(blk);
#pragma unroll
        for (int p = 0; p < 4; p++) wq[p] = ldg16(blk + QO + 32 * p + 16 * h);
        if constexpr (k5) wx = ldg16(blk + 16 + 16 * h); // qh bytes 16h.. (this lane's weights)
    };

    v16f acc[Q2_TT];
#pragma unroll
    for (int t = 0; t < Q2_TT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.0f;

    // Output: y[token][row], bias, accumulate. Each token tile is stored as soon as the last
    // super-block has finished it, so its stores overlap the next tiles' MFMAs.
    const float bias_r = (a.bias && myrow < a.rows) ? a.bias[myrow] : 0.0f;
    const uint32_t rw0 = r0 + 32 * wave;
    auto store_tile = [&](int t) {
        const uint32_t tk0 = t0 + 32 * t;
        if (a.wide && rw0 + 32 <= a.rows && tk0 + 32 <= a.n)
            gemm_store_tile_wide(S.st[wave], acc[t], bias_r, a.y, a.rows, rw0, tk0, a.mode);
        else
            gemm_store_tile(acc[t], bias_r, a.y, a.rows, a.n, myrow, tk0, a.mode);
    };

    stage_load(0, 0);
    wload(0);
    stage_store(0);
    __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): the direct-to-LDS loads have landed
    __syncthreads();

    // One super-block; the last one (LAST) loads nothing ahead and stores each finished tile.
    auto step = [&](uint32_t sb, auto last_c) {
        constexpr bool LAST = decltype(last_c)::value;
        const uint32_t buf = sb & 1;
        const uint4 ch = wh, c0 = wq[0], c1 = wq[1], c2 = wq[2], c3 = wq[3], cx = wx;
        const uint32_t nx = sb + 1;
        if constexpr (!LAST) stage_load(nx, buf ^ 1);

        // Unpack: scales (vecdot.zig:461-474 word form), then both planes of the 8 sub-blocks.
        const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
        const uint32_t scl = ch.y & k1, mnl = ch.z & k1;
        const uint32_t sch = (ch.w & k2) | (((ch.y >> 6) & k3) << 4);
        const uint32_t mnh = ((ch.w >> 4) & k2) | (((ch.z >> 6) & k3) << 4);
        const float d = f16_bits_to_f32(ch.x & 0xFFFF), dmin = f16_bits_to_f32(ch.x >> 16);
        v4i bhi[8], blo[8];
        const uint4 cq[4] = {c0, c1, c2, c3};
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint32_t se = (p < 2 ? scl >> (16 * p) : sch >> (16 * (p - 2))) & 0xFF;
            const uint32_t so = (p < 2 ? scl >> (16 * p + 8) : sch >> (16 * (p - 2) + 8)) & 0xFF;
            const uint32_t she = (se >> 3) * 0x00010001u, sle = (se & 7) * 0x00010001u;
            const uint32_t sho = (so >> 3) * 0x00010001u, slo = (so & 7) * 0x00010001u;
            const uint32_t qw[4] = {cq[p].x, cq[p].y, cq[p].z, cq[p].w};
            const uint32_t xw[4] = {cx.x, cx.y, cx.z, cx.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t ne = qw[i] & 0x0F0F0F0Fu, no = (qw[i] >> 4) & 0x0F0F0F0Fu;
                if constexpr (k5) {
                    // Fifth bits: bit 2p (low nibbles) / 2p + 1 (high) of qh (k4Block has_high).
                    const uint32_t ue = ne | (((xw[i] >> (2 * p)) & 0x01010101u) << 4);
                    const uint32_t uo = no | (((xw[i] >> (2 * p + 1)) & 0x01010101u) << 4);
                    const uint32_t ee = ue & 0x00FF00FFu, eo = (ue >> 8) & 0x00FF00FFu;
                    const uint32_t oe = uo & 0x00FF00FFu, oo = (uo >> 8) & 0x00FF00FFu;
                    bhi[2 * p][i] = int(plane_c16(ee, eo, she, neg16(she)));
                    blo[2 * p][i] = int(plane_c16(ee, eo, sle, neg16(sle)));
                    bhi[2 * p + 1][i] = int(plane_c16(oe, oo, sho, neg16(sho)));
                    blo[2 * p + 1][i] = int(plane_c16(oe, oo, slo, neg16(slo)));
                } else {
                    bhi[2 * p][i] = int(mul_bytes(ne, she));
                    blo[2 * p][i] = int(mul_bytes(ne, sle));
                    bhi[2 * p + 1][i] = int(mul_bytes(no, sho));
                    blo[2 * p + 1][i] = int(mul_bytes(no, slo));
                }
            }
        }
        // Min-term operands of this lane's row.
        MinB mB;
        if constexpr (k5)
            mB = min_operands_k5(scl, sch, d, mnl, mnh, dmin, h);
        else
            mB = min_operands(mnl, mnh, dmin, h);

        // A operand of tile t, sub-block s: token 32t + j, chunk 2s + h (swizzled).
        const int8_t *abase = &S.a[buf][j * 256];
        const uint32_t sw = j & 15;
        v4i av[8];
        auto load_a = [&](int t) {
#pragma unroll
            for (int s = 0; s < 8; s++)
                av[s] = *reinterpret_cast<const v4i *>(abase + 32 * t * 256 + 16 * ((2 * s + h) ^ sw));
        };
        load_a(0);
#pragma unroll
        for (int t = 0; t < Q2_TT; t++) {
            // One accumulator: the sh-plane chain, times 8, then the sl-plane chain on top.
            v16i sacc = {};
#pragma unroll
            for (int s = 0; s < 8; s++) sacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[s], bhi[s], sacc, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; v++) sacc[v] <<= 3;
#pragma unroll
            for (int s = 0; s < 8; s++) sacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[s], blo[s], sacc, 0, 0, 0);
            if (t + 1 < Q2_TT) load_a(t + 1);
            if constexpr (!LAST)
                if (t == (Q2_TT > 1 ? 1 : 0)) wload(nx); // next super-block's weights, once this one's raw words are dead
            // Token scales of this lane's 16 outputs: tokens 32t + 8g + 4h + (0..3).
            const float4 *dap = reinterpret_cast<const float4 *>(&S.da[buf][32 * t + 4 * h]);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 dv = dap[2 * g];
                const float ds[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int v = 4 * g + e;
                    acc[t][v] = fmaf((float)sacc[v], d * ds[e], acc[t][v]);
                }
            }
            // Min term: tokens' da*bsum32 (A) x rows' -dmin*mn (B), bf16 hi/lo split.
            min_term(acc[t], S.mb[buf][32 * t + j], mB, h);
            if constexpr (LAST) store_tile(t);
        }

        if constexpr (!LAST) {
            stage_store(buf ^ 1);
            __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): next super-block's activations are in LDS
            __syncthreads();
        }
    };
    for (uint32_t sb = 0; sb + 1 < nsb; sb++) step(sb, std::false_type{});
    step(nsb - 1, std::true_type{});
}



// KS > 1 splits K: the workgroup's waves form KS slices of NW waves; slice k takes super-blocks
// k, k + KS, ... through a ring of its own, and the slices' partial tiles are added in LDS (in
// slice order) at the end. For matrices too small to give every SIMD two waves otherwise.
template <int NW, int TT, int NB, int KS = 1, int T = HKHIP_Q4_K>
__global__ __launch_bounds__(NW * KS * 64, 2) void mm2_q4k_kernel(Mm2Args a) {
    constexpr int ROWS = 32 * NW, TOK = 32 * TT;
    // Q5_K: 176-byte rows (5 x 1 KB + 512 B per wave and step), the register tile's planes and
    // a second exact integer, Jsc = sum sc*bsum32, for the 16*sum(sc*a) the planes' u - 16 removes.
    constexpr bool k5 = (T == HKHIP_Q5_K);
    constexpr uint32_t BB = k5 ? 176 : 144, PR = BB / 16, WR = BB / 4, W16 = k5 ? 5 : 4, QO = k5 ? 48 : 16;
    using Slot = Q2Slot<TOK, NW, 32 * BB>;
    static_assert(NB == 2 || NB == 3, "ring depth");
    // The ring's slots are LDS objects of their own, and the loop below is unrolled over them.
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

    // Workgroup -> (row block, token block). The token blocks of one row block are consecutive
    // workgroups on the same XCD (workgroups go round-robin over the 8 XCDs), so the rows they
    // share are read from HBM once and then served by that XCD's L2.
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
    const uint32_t r0 = rb * ROWS, t0 = tb * TOK;
    const uint32_t myrow = r0 + 32 * wave + j;

    // ---- the direct loads of one super-block into a slot (CPW per wave) ----
    constexpr uint32_t TPW = TOK / NW; // token rows per wave
    static_assert(TPW % 4 == 0, "token rows per wave");
    constexpr uint32_t CPW = TPW / 4 + W16 + 2 + 1 + 1; // a + w + mb + da
    // Weight bytes of this wave: 16-byte piece P (64*i + lane, i < 4) is byte 16*(P%9) of row
    // P/9's block; the last 512 bytes (pieces 256..287) go as 4-byte words 1024 + 64*i + lane.
    // Per-lane 32-bit byte offsets from uniform bases (mm2_supports checks that they fit).
    uint32_t woff[W16 + 2];
#pragma unroll
    for (uint32_t i = 0; i < W16; i++) {
        const uint32_t P = 64 * i + lane;
        const uint32_t row = r0 + 32 * wave + P / PR, rr = row < a.rows ? row : a.rows - 1;
        woff[i] = rr * nsb * BB + 16 * (P % PR);
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t Wd = 256 * W16 + 64 * i + lane; // 4-byte word index in the wave's area
        const uint32_t row = r0 + 32 * wave + Wd / WR, rr = row < a.rows ? row : a.rows - 1;
        woff[W16 + i] = rr * nsb * BB + 4 * (Wd % WR);
    }
    uint32_t aoff[TPW / 4];
#pragma unroll
    for (uint32_t i = 0; i < TPW / 4; i++) {
        const uint32_t tl = TPW * wave + 4 * i + lane / 16;
        const uint32_t c = (lane % 16) ^ (tl & 15);
        const uint32_t tok = t0 + tl, tk = tok < a.n ? tok : a.n - 1;
        aoff[i] = tk * K + 16 * c;
    }
    auto issue = [&](uint32_t sb, Slot &S) {
        const int8_t *ga = a.aqs + 256 * sb;
#pragma unroll
        for (uint32_t i = 0; i < TPW / 4; i++) load_lds16(ga + aoff[i], &S.a[(TPW * wave + 4 * i) * 256]);
        const uint8_t *gw = a.w + uint64_t(sb) * BB;
#pragma unroll
        for (uint32_t i = 0; i < W16; i++) load_lds16(gw + woff[i], &S.w[wave][1024 * i]);
#pragma unroll
        for (int i = 0; i < 2; i++) load_lds4(gw + woff[W16 + i], &S.w[wave][1024 * W16 + 256 * i]);
        {
            const uint32_t tl = 32 * wave + lane / 2, tok = t0 + (tl < TOK ? tl : 0);
            const uint32_t tk = tok < a.n ? tok : a.n - 1;
            load_lds16(a.amb + (uint64_t(tk) * nsb + sb) * 32 + 16 * (lane & 1), &S.mb[32 * wave][0]);
        }
        {
            const uint32_t tl = 64 * wave + lane, tok = t0 + (tl < TOK ? tl : 0);
            const uint32_t tk = tok < a.n ? tok : a.n - 1;
            load_lds4(a.ad + uint64_t(tk) * nsb + sb, &S.da[64 * wave]);
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

    // Prologue: NB-1 super-blocks in flight.
    issue(sb_of(0), slot_at(std::integral_constant<int, 0>{}));
    if constexpr (NB == 3) issue(sb_of(1), slot_at(std::integral_constant<int, 1>{}));
    // Wait for slot 0 (the loads of NB-2 later super-blocks may stay in flight).
    __builtin_amdgcn_s_waitcnt((0x0F70 & ~0xF) | ((CPW * (NB - 2)) & 0xF) | (((CPW * (NB - 2)) >> 4) << 14));
    __syncthreads();

    // One super-block from slot IC while the one NB-1 ahead goes into slot (IC + NB-1) % NB.
    auto step = [&](auto ic, uint32_t st) {
        constexpr int I = decltype(ic)::value;
        issue(sb_of(st + NB - 1), slot_at(std::integral_constant<int, (I + NB - 1) % NB>{}));
        Slot &S = slot_at(ic);
        if (KS == 1 || ks + KS * st < nsb) {
            // Unpack this lane's row half (h) from LDS: header, then both planes of 8 sub-blocks.
            const uint8_t *blk = &S.w[wave][BB * j];
            const uint4 ch = *reinterpret_cast<const uint4 *>(blk);
            uint4 cq[4], cx{};
#pragma unroll
            for (int p = 0; p < 4; p++) cq[p] = *reinterpret_cast<const uint4 *>(blk + QO + 32 * p + 16 * h);
            if constexpr (k5) cx = *reinterpret_cast<const uint4 *>(blk + 16 + 16 * h);
            // Scales: vecdot.zig:461-474 word form.
            const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
            const uint32_t scl = ch.y & k1, mnl = ch.z & k1;
            const uint32_t sch = (ch.w & k2) | (((ch.y >> 6) & k3) << 4);
            const uint32_t mnh = ((ch.w >> 4) & k2) | (((ch.z >> 6) & k3) << 4);
            const float d = f16_bits_to_f32(ch.x & 0xFFFF), dmin = f16_bits_to_f32(ch.x >> 16);
            v4i bhi[8], blo[8];
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const uint32_t se = (p < 2 ? scl >> (16 * p) : sch >> (16 * (p - 2))) & 0xFF;
                const uint32_t so = (p < 2 ? scl >> (16 * p + 8) : sch >> (16 * (p - 2) + 8)) & 0xFF;
                const uint32_t she = (se >> 3) * 0x00010001u, sle = (se & 7) * 0x00010001u;
                const uint32_t sho = (so >> 3) * 0x00010001u, slo = (so & 7) * 0x00010001u;
                const uint32_t qw[4] = {cq[p].x, cq[p].y, cq[p].z, cq[p].w};
                const uint32_t xw[4] = {cx.x, cx.y, cx.z, cx.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t ne = qw[i] & 0x0F0F0F0Fu, no = (qw[i] >> 4) & 0x0F0F0F0Fu;
                    if constexpr (k5) {
                        const uint32_t ue = ne | (((xw[i] >> (2 * p)) & 0x01010101u) << 4);
                        const uint32_t uo = no | (((xw[i] >> (2 * p + 1)) & 0x01010101u) << 4);
                        const uint32_t ee = ue & 0x00FF00FFu, eo = (ue >> 8) & 0x00FF00FFu;
                        const uint32_t oe = uo & 0x00FF00FFu, oo = (uo >> 8) & 0x00FF00FFu;
                        bhi[2 * p][i] = int(plane_c16(ee, eo, she, neg16(she)));
                        blo[2 * p][i] = int(plane_c16(ee, eo, sle, neg16(sle)));
                        bhi[2 * p + 1][i] = int(plane_c16(oe, oo, sho, neg16(sho)));
                        blo[2 * p + 1][i] = int(plane_c16(oe, oo, slo, neg16(slo)));
                    } else {
                        bhi[2 * p][i] = int(mul_bytes(ne, she));
                        blo[2 * p][i] = int(mul_bytes(ne, sle));
                        bhi[2 * p + 1][i] = int(mul_bytes(no, sho));
                        blo[2 * p + 1][i] = int(mul_bytes(no, slo));
                    }
                }
            }
            // Min-term operand of this lane's row.
            const v8bf mB = min_b(mnl, mnh);
            const v8bf sB = k5 ? min_b(scl, sch) : mB; // Q5_K: the scales as exact bf16 integers
            const float ndmin = -dmin;

            // A operand of tile t, sub-block s: token 32t + j, chunk 2s + h (swizzled).
            const int8_t *abase = &S.a[j * 256];
            const uint32_t sw = j & 15;
            v4i av[8];
            auto load_a = [&](int t) {
#pragma unroll
                for (int s = 0; s < 8; s++)
                    av[s] = *reinterpret_cast<const v4i *>(abase + 32 * t * 256 + 16 * ((2 * s + h) ^ sw));
            };
            load_a(0);
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const v16f jt = min_j(S.mb[32 * t + j], mB, h, acc[t][15]);
                v16f js = {};
                if constexpr (k5) js = min_j(S.mb[32 * t + j], sB, h, jt[15]);
                // One accumulator: the sh-plane chain, times 8, then the sl-plane chain on top.
                v16i sacc = {};
#pragma unroll
                for (int s = 0; s < 8; s++) sacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[s], bhi[s], sacc, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; v++) sacc[v] <<= 3;
#pragma unroll
                for (int s = 0; s < 8; s++) sacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[s], blo[s], sacc, 0, 0, 0);
                if (t + 1 < TT) load_a(t + 1);
                // Token scales of this lane's 16 outputs: tokens 32t + 8g + 4h + (0..3).
                const float4 *dap = reinterpret_cast<const float4 *>(&S.da[32 * t + 4 * h]);
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const float4 dv = dap[2 * g];
                    const float ds[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int v = 4 * g + e;
                        const float iv = k5 ? fmaf(16.0f, js[v], (float)sacc[v]) : (float)sacc[v];
                        acc[t][v] = fmaf(fmaf(iv, d, ndmin * jt[v]), ds[e], acc[t][v]);
                    }
                }
            }
        }
        // The next super-block's slot has landed once at most NB-2 later issues are pending.
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

bool mm2_supports(int t, uint32_t rows, uint32_t cols, uint32_t n) {
    // The kernels' per-lane byte offsets are 32-bit: weights rows*cols*9/16 bytes, activations
    // n*cols bytes.
    if (t == HKHIP_Q5_K) // the register tile and the 128-row ring tile, where they fill the GPU
        return cols % 256 == 0 &&
               (((rows + 255) / 256) * ((n + 127) / 128) >= 192 || ((rows + 127) / 128) * ((n + 63) / 64) >= 160) &&
               uint64_t(rows) * (cols / 256) * 176 < (1ull << 32) && uint64_t(n) * cols < (1ull << 32);
    return t == HKHIP_Q4_K && cols % 256 == 0 && rows > 0 && n > 0 &&
           uint64_t(rows) * (cols / 256) * 144 < (1ull << 32) && uint64_t(n) * cols < (1ull << 32);
}

typedef void (*mm2_kernel_t)(Mm2Args);

template <int NW, int TT, int T = HKHIP_Q4_K>
static hipError_t launch_mm2_reg(const Mm2Args &a0, hipStream_t s) {
    const mm2_kernel_t k = mm2_q4k_reg_kernel<T, NW, TT>;
    constexpr size_t lds = sizeof(Q2Smem<32 * TT, NW>);
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        attr = true;
    }
    Mm2Args a = a0;
    a.rblocks = (a.rows + 32 * NW - 1) / (32 * NW);
    a.tblocks = (a.n + 32 * TT - 1) / (32 * TT);
    hipLaunchKernelGGL(k, dim3(a.rblocks * a.tblocks), dim3(NW * 64), lds, s, a);
    return hipGetLastError();
}

template <int NW, int TT, int NB, int KS = 1, int T = HKHIP_Q4_K>
static hipError_t launch_mm2_cfg(const Mm2Args &a0, hipStream_t s) {
    const mm2_kernel_t k = mm2_q4k_kernel<NW, TT, NB, KS, T>;
    static_assert(NB * KS * sizeof(Q2Slot<32 * TT, NW, T == HKHIP_Q5_K ? 5632 : 4608>) <= 160 * 1024, "LDS");
    constexpr size_t lds = 0; // the ring is static
    Mm2Args a = a0;
    a.rblocks = (a.rows + 32 * NW - 1) / (32 * NW);
    a.tblocks = (a.n + 32 * TT - 1) / (32 * TT);
    hipLaunchKernelGGL(k, dim3(a.rblocks * a.tblocks), dim3(NW * KS * 64), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_mm2(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n, float *y,
                      const float *bias, int mode, hipStream_t s) {
    if (!mm2_supports(t, rows, cols, n)) return hipErrorInvalidValue;
    const ActLayout A = act_layout(n, cols);
    Mm2Args a{};
    a.w = w;
    a.rows = rows;
    a.cols = cols;
    a.n = n;
    a.aqs = reinterpret_cast<const int8_t *>(xq + A.k_qs);
    a.ad = reinterpret_cast<const float *>(xq + A.k_d);
    a.abs = reinterpret_cast<const int16_t *>(xq + A.k_bs);
    a.amb = xq + A.k_mb;
    a.y = y;
    a.bias = bias;
    a.mode = mode;
    a.wide = (reinterpret_cast<uintptr_t>(y) % 16 == 0 && rows % (mode == HKHIP_SILU_MUL ? 8 : 4) == 0) ? 1 : 0;
    // The largest tile that still gives most of the 256 CUs a workgroup.
    auto blocks = [&](uint32_t nw, uint32_t tt) {
        return ((rows + 32 * nw - 1) / (32 * nw)) * ((n + 32 * tt - 1) / (32 * tt));
    };
    // Below that, K slices give the SIMDs a second wave (measured at 512 tokens: 4096x14336
    // 104 -> 87 us with two slices, 1024x3072 16.8 -> 10.7 us with four).
    const uint32_t nsb = cols / 256;
    if (t == HKHIP_Q5_K) // mm2_supports: these two tiles only (two K slices would not fit the LDS)
        return blocks(8, 4) >= 192 ? launch_mm2_reg<8, 4, HKHIP_Q5_K>(a, s) : launch_mm2_cfg<4, 2, 2, 1, HKHIP_Q5_K>(a, s);
    if (blocks(8, 4) >= 192) return launch_mm2_reg<8, 4>(a, s);
    // Two K slices only while the grid stays within one workgroup per CU: a 512-thread workgroup
    // leaves no room for a second, so past 256 the grid runs in two rounds (6144x1024 at 512
    // tokens: 19.1 us with two slices, 15.9 with one).
    if (blocks(4, 2) >= 160)
        return nsb >= 4 && blocks(4, 2) <= 256 ? launch_mm2_cfg<4, 2, 2, 2>(a, s) : launch_mm2_cfg<4, 2, 2>(a, s);
    if (blocks(2, 1) >= 128) {
        if (nsb >= 8) return launch_mm2_cfg<2, 1, 2, 4>(a, s);
        if (nsb >= 2) return launch_mm2_cfg<2, 1, 2, 2>(a, s);
        return launch_mm2_cfg<2, 1, 3>(a, s);
    }
    return launch_mm2_cfg<1, 1, 3>(a, s);
}

} // namespace hkhip
