// The formats hk decodes to floats before its dot products ("exact fallback"): Q2_K, Q3_K,
// IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, TQ1_0, TQ2_0, MXFP4, NVFP4.
//
// Decoders restate src/quant/dequant.zig (q2_k 80-112, q3kScales 114-128, q3_k 130-165,
// iq2_xxs 278-294, iq2_xs 296-312, iq2_s 314-330, iq3_xxs 332-351, iq3_s 353-375, iq1_s 377-392,
// iq1_m 394-428, ternary / tq1_0 460-488, tq2_0 490-504, e8m0Half / mxfp4 506-519, ue4m3Half /
// nvfp4 521-548) one element at a time with the reference's float operations in its order (the
// library is built with -ffp-contract=off), so they are bit-exact. The device layout is the file
// layout. Products follow hk's fallback dots (vecdot.zig dotCanonK 686-705, dotCanonLegacy 707-720,
// dotGeneric 620-631): the weights against the dequantized Q8K / A8 activations (d * q), or the f32
// input for NVFP4, summed in f32 -- the integer dot of the reference up to rounding.
//
// Products: a wave owns up to FB_RPW output rows (pairs of rows for silu(gate)*up); for every
// 256 inputs it first forms its lanes' four activation values per token (reading a prepared
// buffer, or quantizing the f32 input itself with the qact arithmetic: a Q8K block is the whole
// wave, an A8 block eight lanes), then decodes four weights of each of its rows per lane.
#include "quant.hpp"
#include "iq_tables.inc" // the IQ codebooks (hk_amd/csrc/tables/*.bin) as __constant__ arrays

namespace hkhip {
namespace {

__device__ __forceinline__ float ldh(const uint8_t *p) { return f16_bits_to_f32(uint32_t(p[0]) | (uint32_t(p[1]) << 8)); }
__device__ __forceinline__ uint32_t ld32(const uint8_t *p) {
    return uint32_t(p[0]) | (uint32_t(p[1]) << 8) | (uint32_t(p[2]) << 16) | (uint32_t(p[3]) << 24);
}
__device__ __forceinline__ uint32_t ld16(const uint8_t *p) { return uint32_t(p[0]) | (uint32_t(p[1]) << 8); }
// ksigns_iq2xs: seven sign bits plus an eighth that makes their count even.
__device__ __forceinline__ uint32_t ksign(uint32_t i) { return i | ((__popc(i) & 1u) << 7); }
__device__ __forceinline__ float sgn(uint32_t s, uint32_t j) { return (s >> j) & 1u ? -1.0f : 1.0f; }
__device__ __forceinline__ float fp4v(uint32_t nib) { // tables.zig:16 kvalues_fp4
    const int v[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    return float(v[nib & 15]);
}
constexpr float IQ1S_DELTA = 0.125f; // tables.zig:18

// Element e of one block.
__device__ float fb_elem(int t, const uint8_t *b, uint32_t e) {
    switch (t) {
    case HKHIP_Q2_K: { // {scales[16], qs[64], d, dmin}
        const uint32_t n = e / 128, it = (e % 128) / 32, half = (e % 32) / 16, l = e % 16;
        const uint32_t sc = b[8 * n + 2 * it + half];
        const float d = ldh(b + 80), mn = ldh(b + 82);
        const float dl = d * float(sc & 0x0F), ml = mn * float(sc >> 4);
        return dl * float((b[16 + 32 * n + 16 * half + l] >> (2 * it)) & 3) - ml;
    }
    case HKHIP_Q3_K: { // {hmask[32], qs[64], scales[12], d}
        const uint32_t n = e / 128, it = (e % 128) / 32, half = (e % 32) / 16, l = e % 16;
        const uint32_t is = 8 * n + 2 * it + half; // scale index 0..15 (q3kScales)
        const uint32_t a0 = ld32(b + 96), a1 = ld32(b + 100), tmp = ld32(b + 104);
        uint32_t word;
        switch (is / 4) {
        case 0: word = (a0 & 0x0f0f0f0fu) | (((tmp >> 0) & 0x03030303u) << 4); break;
        case 1: word = (a1 & 0x0f0f0f0fu) | (((tmp >> 2) & 0x03030303u) << 4); break;
        case 2: word = ((a0 >> 4) & 0x0f0f0f0fu) | (((tmp >> 4) & 0x03030303u) << 4); break;
        default: word = ((a1 >> 4) & 0x0f0f0f0fu) | (((tmp >> 6) & 0x03030303u) << 4); break;
        }
        const int sc = int(int8_t(uint8_t(word >> (8 * (is % 4)))));
        const float dl = ldh(b + 108) * float(sc - 32);
        const int lo = (b[32 + 32 * n + 16 * half + l] >> (2 * it)) & 3;
        const int hi = (b[16 * half + l] & (1u << (4 * n + it))) ? 0 : 4;
        return dl * float(lo - hi);
    }
    case HKHIP_IQ2_XXS: { // {d, qs[64]}
        const uint32_t ib = e / 32, l = (e % 32) / 8, j = e % 8;
        const uint32_t aux1 = ld32(b + 2 + 8 * ib + 4);
        const float db = ldh(b) * (0.5f + float(aux1 >> 28)) * 0.25f;
        const uint32_t g = iq2xxs_grid[8 * b[2 + 8 * ib + l] + j];
        return db * float(g) * sgn(ksign((aux1 >> (7 * l)) & 127), j);
    }
    case HKHIP_IQ2_XS: { // {d, qs[32] u16, scales[8]}
        const uint32_t ib = e / 32, l = (e % 32) / 8, j = e % 8;
        const uint32_t sc = b[66 + ib];
        const float d = ldh(b);
        const float db = l < 2 ? d * (0.5f + float(sc & 0x0F)) * 0.25f : d * (0.5f + float(sc >> 4)) * 0.25f;
        const uint32_t q = ld16(b + 2 + 2 * (4 * ib + l));
        return db * float(iq2xs_grid[8 * (q & 511) + j]) * sgn(ksign(q >> 9), j);
    }
    case HKHIP_IQ2_S: { // {d, qs[32], signs[32], qh[8], scales[8]}
        const uint32_t ib = e / 32, l = (e % 32) / 8, j = e % 8;
        const uint32_t sc = b[74 + ib];
        const float d = ldh(b);
        const float db = l < 2 ? d * (0.5f + float(sc & 0x0F)) * 0.25f : d * (0.5f + float(sc >> 4)) * 0.25f;
        const uint32_t hi = (uint32_t(b[66 + ib]) << (8 - 2 * l)) & 0x300;
        return db * float(iq2s_grid[8 * (b[2 + 4 * ib + l] | hi) + j]) * sgn(b[34 + 4 * ib + l], j);
    }
    case HKHIP_IQ3_XXS: { // {d, qs[96]}
        const uint32_t ib = e / 32, l = (e % 32) / 8, j = e % 8;
        const uint32_t aux = ld32(b + 2 + 64 + 4 * ib);
        const float db = ldh(b) * (0.5f + float(aux >> 28)) * 0.5f;
        const uint32_t gi = b[2 + 8 * ib + 2 * l + (j >= 4 ? 1 : 0)];
        return db * float(iq3xxs_grid[4 * gi + (j & 3)]) * sgn(ksign((aux >> (7 * l)) & 127), j);
    }
    case HKHIP_IQ3_S: { // {d, qs[64], qh[8], signs[32], scales[4]}
        const uint32_t g = e / 8, j = e % 8;
        const uint32_t nib = (b[106 + g / 8] >> (4 * ((g / 4) & 1))) & 0x0F;
        const float db = ldh(b) * float(1 + 2 * nib);
        const uint32_t ei = 2 * g + (j >= 4 ? 1 : 0);
        const uint32_t idx = b[2 + ei] | (((uint32_t(b[66 + ei / 8]) >> (ei % 8)) & 1u) << 8);
        return db * float(iq3s_grid[4 * idx + (j & 3)]) * sgn(b[74 + g], j);
    }
    case HKHIP_IQ1_S: { // {d, qs[32], qh[16]}
        const uint32_t ib = e / 32, l = (e % 32) / 8, j = e % 8;
        const uint32_t qh = ld16(b + 34 + 2 * ib);
        const float dl = ldh(b) * float(2 * ((qh >> 12) & 7) + 1);
        const float delta = (qh & 0x8000) ? -IQ1S_DELTA : IQ1S_DELTA;
        const uint32_t idx = b[2 + 4 * ib + l] | (((qh >> (3 * l)) & 7u) << 8);
        return dl * (float(int8_t(iq1s_grid[8 * idx + j])) + delta);
    }
    case HKHIP_IQ1_M: { // {qs[32], qh[16], scales[8]}
        const uint32_t ib = e / 32, l = (e % 32) / 8, j = e % 8;
        const uint32_t s0 = ld16(b + 48), s1 = ld16(b + 50), s2 = ld16(b + 52), s3 = ld16(b + 54);
        const uint32_t bits = (s0 >> 12) | ((s1 >> 8) & 0x00F0) | ((s2 >> 4) & 0x0F00) | (s3 & 0xF000);
        const float d = f16_bits_to_f32(bits);
        const uint32_t w = ld16(b + 48 + 2 * (ib / 2)), base = 6 * (ib % 2);
        const float dl = l < 2 ? d * float(2 * ((w >> base) & 7) + 1) : d * float(2 * ((w >> (base + 3)) & 7) + 1);
        const uint32_t qhb = b[32 + 2 * ib + l / 2];
        const uint32_t idx = b[4 * ib + l] | ((l & 1) ? ((qhb << 4) & 0x700) : ((qhb << 8) & 0x700));
        const float delta = (qhb & ((l & 1) ? 0x80 : 0x08)) ? -IQ1S_DELTA : IQ1S_DELTA;
        return dl * (float(int8_t(iq1s_grid[8 * idx + j])) + delta);
    }
    case HKHIP_TQ1_0: { // {qs[48], qh[4], d}: base-3 digits, five per byte (four in qh)
        uint32_t byte, n;
        if (e < 160) {
            n = e / 32;
            byte = b[e % 32];
        } else if (e < 240) {
            n = (e - 160) / 16;
            byte = b[32 + (e - 160) % 16];
        } else {
            n = (e - 240) / 4;
            byte = b[48 + (e - 240) % 4];
        }
        const uint32_t pow3[5] = {1, 3, 9, 27, 81};
        const uint32_t v = (byte * pow3[n]) & 0xFF;
        const float tv = float(int((v * 3) >> 8) - 1);
        return tv * ldh(b + 52);
    }
    case HKHIP_TQ2_0: { // {qs[64], d}
        const uint32_t j = (e / 128) * 32, l = (e % 128) / 32, k = e % 32;
        return float(int((b[j + k] >> (2 * l)) & 3) - 1) * ldh(b + 64);
    }
    case HKHIP_MXFP4: { // {e, qs[16]}
        const uint32_t x = b[0];
        const float d = __uint_as_float(x < 2 ? (0x00200000u << x) : (x - 1) << 23);
        const uint32_t q = b[1 + (e % 16)];
        return fp4v(e < 16 ? q & 0x0F : q >> 4) * d;
    }
    case HKHIP_NVFP4: { // {d[4], qs[32]}: four 16-value sub-blocks with an unsigned E4M3 scale
        const uint32_t s = e / 16, j = e % 16;
        const uint32_t x = b[s];
        float d = 0.0f;
        if (x != 0 && x != 0x7F) {
            const uint32_t ex = (x >> 3) & 0xF;
            const float man = float(x & 7);
            const float raw = ex == 0 ? man * 0x1p-9f : (1.0f + man / 8.0f) * __uint_as_float((ex - 7 + 127) << 23);
            d = raw * 0.5f;
        }
        const uint32_t q = b[4 + 8 * s + (j % 8)];
        return fp4v(j < 8 ? q & 0x0F : q >> 4) * d;
    }
    default: return 0.0f;
    }
}

__global__ void fb_dequant_kernel(int t, const uint8_t *__restrict__ w, uint32_t cols, uint32_t row0,
                                  const uint32_t *__restrict__ ids, uint64_t total, float *__restrict__ out) {
    const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const uint64_t r = ids ? uint64_t(ids[i / cols]) : row0 + i / cols;
    const uint32_t c = uint32_t(i % cols), el = uint32_t(block_elems(t));
    const uint8_t *blk = w + (r * (cols / el) + c / el) * uint64_t(block_bytes(t));
    out[i] = fb_elem(t, blk, c % el);
}

constexpr int FB_RPW = 8; // output rows per wave
constexpr int FB_NW = 4;  // waves per workgroup

struct FbPart {
    const uint8_t *w;
    float *y;
    const float *bias;
    uint32_t rows, ustart; // ustart: first output unit of this part
};
struct FbArgs {
    FbPart p[4];
    uint32_t nparts, units, K, ntok;
    int t, mode;
    const float *x;   // f32 input [ntok][K], or null
    const int8_t *qs; // prepared activations (A8 or Q8K planes)
    const float *d;
};

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// The four activation values a lane uses at inputs e0..e0+3 of token t (e0 = 256*g + 4*lane):
// d * q of the prepared buffer, or the qact arithmetic applied to the f32 input right here.
template <int KIND>
__device__ __forceinline__ void fb_acts(const FbArgs &a, uint32_t t, uint32_t g, float out[4]) {
    const uint32_t lane = __lane_id(), K = a.K, e0 = 256 * g + 4 * lane;
    if constexpr (KIND == HKHIP_ACT_F32) {
        const float4 v = *reinterpret_cast<const float4 *>(a.x + uint64_t(t) * K + e0);
        out[0] = v.x, out[1] = v.y, out[2] = v.z, out[3] = v.w;
    } else if (a.x == nullptr) {
        const uint32_t q = *reinterpret_cast<const uint32_t *>(a.qs + uint64_t(t) * K + e0);
        const float d = a.d[(uint64_t(t) * K + e0) / (KIND == HKHIP_ACT_Q8K ? 256 : 32)];
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = d * float(int8_t(uint8_t(q >> (8 * i))));
    } else {
        const float4 v4 = *reinterpret_cast<const float4 *>(a.x + uint64_t(t) * K + e0);
        const float v[4] = {v4.x, v4.y, v4.z, v4.w};
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) m = fmaxf(m, fabsf(v[i]));
        if constexpr (KIND == HKHIP_ACT_Q8K) {
            // quantizeQ8K (vecdot.zig:150-180): the signed value of the first element with the
            // largest magnitude sets the scale; q = min(127, round(iscale * x)); d = 1 / iscale.
            const float amax = wave_max(m);
            int first = 4;
#pragma unroll
            for (int i = 3; i >= 0; i--)
                if (fabsf(v[i]) == amax) first = i;
            const uint64_t hit = __ballot(first < 4);
            const uint32_t src = hit ? uint32_t(__builtin_ctzll(hit)) : 0u;
            const float mine = first < 4 ? v[first < 4 ? first : 0] : 0.0f;
            const float mx = __shfl(mine, int(src));
            const bool zero = amax == 0.0f;
            const float iscale = zero ? 0.0f : __fdiv_rn(-127.0f, mx);
            const float d = zero ? 0.0f : __fdiv_rn(1.0f, iscale);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int q = int(roundf(iscale * v[i]));
                out[i] = d * float(q < 127 ? q : 127);
            }
        } else {
            // quantizeA8 (vecdot.zig:134-148): per 32 inputs (eight lanes) d = amax / 127.
            float am = m;
            for (int o = 1; o <= 4; o <<= 1) am = fmaxf(am, __shfl_xor(am, o));
            const float d = __fdiv_rn(am, 127.0f);
            const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) out[i] = d * float(int(roundf(v[i] * id)));
        }
    }
}

template <int KIND, int NT>
__global__ __launch_bounds__(FB_NW * 64) void fb_mv_kernel(FbArgs a) {
    const uint32_t lane = __lane_id(), wave = threadIdx.x >> 6;
    const uint32_t u0 = (blockIdx.x * FB_NW + wave) * FB_RPW;
    if (u0 >= a.units) return; // whole waves only: the quantizing shuffles need all 64 lanes
    const bool pairs = a.mode == HKHIP_SILU_MUL;
    const uint32_t el = uint32_t(block_elems(a.t)), bb = uint32_t(block_bytes(a.t));
    const uint64_t rowbytes = uint64_t(a.K / el) * bb;
    float acc[FB_RPW][2][NT];
#pragma unroll
    for (int r = 0; r < FB_RPW; r++)
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int t = 0; t < NT; t++) acc[r][h][t] = 0.0f;
    // Output unit u is row u of its part, or rows 2u, 2u + 1 (gate, up) for silu(gate)*up.
    auto part_of = [&](uint32_t u) {
        FbPart q = a.p[0];
#pragma unroll
        for (int i = 1; i < 4; i++)
            if (i < int(a.nparts) && u >= a.p[i].ustart) q = a.p[i];
        return q;
    };
    const uint8_t *rowp[FB_RPW];
#pragma unroll
    for (int r = 0; r < FB_RPW; r++) {
        const uint32_t u = u0 + r < a.units ? u0 + r : a.units - 1;
        const FbPart q = part_of(u);
        rowp[r] = q.w + uint64_t(u - q.ustart) * (pairs ? 2 : 1) * rowbytes;
    }
    for (uint32_t g = 0; g < a.K / 256; g++) {
        float av[NT][4];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (uint32_t(t) < a.ntok)
                fb_acts<KIND>(a, t, g, av[t]);
            else
                av[t][0] = av[t][1] = av[t][2] = av[t][3] = 0.0f;
        }
        const uint32_t e0 = 256 * g + 4 * lane; // four inputs of one block (blocks hold 32..256)
        const uint32_t boff = (e0 / el) * bb, ein = e0 % el;
#pragma unroll
        for (int r = 0; r < FB_RPW; r++) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                if (h == 1 && !pairs) break;
                const uint8_t *blk = rowp[r] + (h ? rowbytes : 0) + boff;
                float wv[4];
#pragma unroll
                for (int i = 0; i < 4; i++) wv[i] = fb_elem(a.t, blk, ein + i);
#pragma unroll
                for (int t = 0; t < NT; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[r][h][t] = fmaf(wv[i], av[t][i], acc[r][h][t]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < FB_RPW; r++) {
        const uint32_t u = u0 + r;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float s0 = acc[r][0][t], s1 = acc[r][1][t];
            for (int o = 32; o >= 1; o >>= 1) {
                s0 += __shfl_xor(s0, o);
                s1 += __shfl_xor(s1, o);
            }
            if (lane == 0 && u < a.units && uint32_t(t) < a.ntok) {
                const FbPart q = part_of(u);
                const uint32_t o = u - q.ustart;
                if (pairs) {
                    q.y[uint64_t(t) * (q.rows / 2) + o] = silu_mul(s0, s1);
                } else {
                    const float b = q.bias ? q.bias[o] : 0.0f;
                    float *y = q.y + uint64_t(t) * q.rows + o;
                    if (a.mode == HKHIP_ACCUMULATE)
                        *y += s0 + b;
                    else
                        *y = s0 + b;
                }
            }
        }
    }
}

template <int KIND>
hipError_t fb_mv_launch(const FbArgs &a, uint32_t nt, hipStream_t s) {
    const dim3 grid((a.units + FB_NW * FB_RPW - 1) / (FB_NW * FB_RPW)), block(FB_NW * 64);
    switch (nt) {
    case 1: hipLaunchKernelGGL((fb_mv_kernel<KIND, 1>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((fb_mv_kernel<KIND, 2>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((fb_mv_kernel<KIND, 4>), grid, block, 0, s, a); break;
    case 8: hipLaunchKernelGGL((fb_mv_kernel<KIND, 8>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

} // namespace
} // namespace hkhip

namespace hkhip {

hipError_t launch_fb_dequant(int t, const uint8_t *w, uint32_t cols, uint32_t row0, const uint32_t *ids, uint32_t nrows,
                             float *out, hipStream_t s) {
    const uint64_t total = uint64_t(nrows) * cols;
    if (total == 0) return hipSuccess;
    const uint64_t grid = (total + 255) / 256;
    if (grid > 0x7fffffffu) return hipErrorInvalidValue;
    hipLaunchKernelGGL(fb_dequant_kernel, dim3(uint32_t(grid)), dim3(256), 0, s, t, w, cols, row0, ids, total, out);
    return hipGetLastError();
}

hipError_t launch_fb_mv(int t, const MvPartDesc *parts, int nparts, uint32_t K, const float *x, const uint8_t *xq,
                        uint32_t n, int mode, hipStream_t s) {
    const int kind = act_kind(t);
    if (n < 1 || nparts < 1 || nparts > 4 || K % 256) return hipErrorInvalidValue;
    if (kind == HKHIP_ACT_F32 && !x) return hipErrorNotSupported;
    FbArgs a{};
    uint32_t units = 0;
    for (int i = 0; i < nparts; i++) {
        a.p[i] = FbPart{parts[i].w, parts[i].y, parts[i].bias, parts[i].rows, units};
        units += mode == HKHIP_SILU_MUL ? parts[i].rows / 2 : parts[i].rows;
    }
    a.nparts = uint32_t(nparts);
    a.units = units;
    a.K = K;
    a.t = t;
    a.mode = mode;
    if (units == 0) return hipSuccess;
    const ActLayout A = act_layout(n, K);
    for (uint32_t t0 = 0; t0 < n; t0 += 8) {
        const uint32_t nc = n - t0 < 8 ? n - t0 : 8;
        FbArgs c = a;
        for (int i = 0; i < nparts; i++)
            c.p[i].y = a.p[i].y + uint64_t(t0) * (mode == HKHIP_SILU_MUL ? a.p[i].rows / 2 : a.p[i].rows);
        c.ntok = nc;
        if (x) {
            c.x = x + uint64_t(t0) * K;
        } else {
            const bool kq = kind == HKHIP_ACT_Q8K;
            c.qs = reinterpret_cast<const int8_t *>(xq + (kq ? A.k_qs : A.a8_qs)) + uint64_t(t0) * K;
            c.d = reinterpret_cast<const float *>(xq + (kq ? A.k_d : A.a8_d)) + uint64_t(t0) * K / (kq ? 256 : 32);
        }
        const uint32_t nt = nc == 1 ? 1 : nc == 2 ? 2 : nc <= 4 ? 4 : 8;
        hipError_t e = kind == HKHIP_ACT_F32 ? fb_mv_launch<HKHIP_ACT_F32>(c, nt, s)
                     : kind == HKHIP_ACT_Q8K ? fb_mv_launch<HKHIP_ACT_Q8K>(c, nt, s)
                                             : fb_mv_launch<HKHIP_ACT_A8>(c, nt, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

} // namespace hkhip
