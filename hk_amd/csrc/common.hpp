// Shared definitions of the HIP engine: device layouts of weights and activations, small
// device helpers, and the launchers each kernel file provides to engine.cpp.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hkhip.h"

// One engine: a device and the stream its work goes to (own: created at init; cur: the one in use).
struct hkhip_engine {
    int device;
    hipStream_t own;
    hipStream_t cur;
    char name[128];
};

namespace hkhip {

// Sets the thread's hkhip_last_error() message and returns code.
int set_error(int code, const char *fmt, ...);

constexpr uint32_t QK_K = 256;

inline uint64_t align256(uint64_t x) { return (x + 255) & ~uint64_t(255); }

// The formats whose products decode the weights to floats (fallback.hip).
__host__ __device__ constexpr bool fallback_type(int t) {
    return t == HKHIP_Q2_K || t == HKHIP_Q3_K || t == HKHIP_IQ2_XXS || t == HKHIP_IQ2_XS || t == HKHIP_IQ2_S ||
           t == HKHIP_IQ3_XXS || t == HKHIP_IQ3_S || t == HKHIP_IQ1_S || t == HKHIP_IQ1_M || t == HKHIP_TQ1_0 ||
           t == HKHIP_TQ2_0 || t == HKHIP_MXFP4 || t == HKHIP_NVFP4;
}

// Block geometry in hk's file layout (src/quant/blocks.zig:13-40).
__host__ __device__ inline int block_elems(int t) {
    switch (t) {
    case HKHIP_Q8_0: case HKHIP_IQ4_NL: case HKHIP_Q4_0: case HKHIP_Q4_1: case HKHIP_Q5_0: case HKHIP_Q5_1:
    case HKHIP_MXFP4:
        return 32;
    case HKHIP_NVFP4: return 64;
    case HKHIP_Q4_K: case HKHIP_Q5_K: case HKHIP_Q6_K: case HKHIP_IQ4_XS: return 256;
    default: return fallback_type(t) ? 256 : 0;
    }
}
__host__ __device__ inline int block_bytes_dev(int t) {
    return t == HKHIP_Q4_0 ? 18 : t == HKHIP_Q4_1 ? 20 : t == HKHIP_Q5_0 ? 22 : t == HKHIP_Q5_1 ? 24 : 0;
}
__host__ __device__ inline int block_bytes(int t) {
    switch (t) {
    case HKHIP_Q2_K: return 84;
    case HKHIP_Q3_K: return 110;
    case HKHIP_IQ2_XXS: return 66;
    case HKHIP_IQ2_XS: return 74;
    case HKHIP_IQ2_S: return 82;
    case HKHIP_IQ3_XXS: return 98;
    case HKHIP_IQ3_S: return 110;
    case HKHIP_IQ1_S: return 50;
    case HKHIP_IQ1_M: return 56;
    case HKHIP_TQ1_0: return 54;
    case HKHIP_TQ2_0: return 66;
    case HKHIP_MXFP4: return 17;
    case HKHIP_NVFP4: return 36;
    case HKHIP_Q8_0: return 34;
    case HKHIP_IQ4_NL: return 18;
    case HKHIP_Q4_K: return 144;
    case HKHIP_Q6_K: return 210;
    case HKHIP_Q5_K: return 176;
    case HKHIP_IQ4_XS: return 136;
    case HKHIP_Q4_0: return 18;
    case HKHIP_Q4_1: return 20;
    case HKHIP_Q5_0: return 22;
    case HKHIP_Q5_1: return 24;
    default: return 0;
    }
}
// vecdot.zig:185-191
inline int act_kind(int t) {
    if (t == HKHIP_NVFP4) return HKHIP_ACT_F32;
    return block_elems(t) == 32 ? HKHIP_ACT_A8 : HKHIP_ACT_Q8K;
}
// The 32-weight formats (A8 activations).
__host__ __device__ constexpr bool legacy32(int t) {
    return t == HKHIP_Q8_0 || t == HKHIP_IQ4_NL || t == HKHIP_Q4_0 || t == HKHIP_Q4_1 || t == HKHIP_Q5_0 ||
           t == HKHIP_Q5_1;
}
// The 4/5-bit 32-weight formats: zero point (gemm.zig:262-270), offset m, fifth bit.
__host__ __device__ constexpr bool has_m(int t) { return t == HKHIP_Q4_1 || t == HKHIP_Q5_1; }
__host__ __device__ constexpr bool has_qh(int t) { return t == HKHIP_Q5_0 || t == HKHIP_Q5_1; }
__host__ __device__ constexpr int zero_point(int t) { return t == HKHIP_Q4_0 ? 8 : t == HKHIP_Q5_0 ? 16 : 0; }
// Geometry of one row's record in the side plane (see WLayout), in bytes: the offsets m and qh
// start at, and the record stride. The fifth-bit words start 4-byte aligned.
struct SideGeom {
    uint32_t m_off, qh_off, stride;
};
__host__ __device__ constexpr SideGeom side_geom(int t, uint32_t nbr) {
    return SideGeom{2 * nbr, ((has_m(t) ? 4 : 2) * nbr + 3) & ~3u,
                    has_qh(t) ? (((has_m(t) ? 4 : 2) * nbr + 3) & ~3u) + 4 * nbr : (has_m(t) ? 4 : 2) * nbr};
}

// Device layout of a weight matrix. Q4_K and Q5_K keep the 144- / 176-byte file blocks (already
// 16-byte aligned). The 2-byte-aligned formats are split at upload into a quant plane whose blocks
// are 16-byte aligned and a plane of f16 scales, one per block, in block order:
//   Q8_0   quant plane: 32 B per block (qs)        scale plane: d
//   IQ4_NL quant plane: 16 B per block (qs)        scale plane: d
//   Q6_K   quant plane: 208 B per block (ql qh sc) scale plane: d
//   IQ4_XS quant plane: 128 B per block (qs)       side plane: the 8-B header (d, scales_h,
//                                                   scales_l), block order
//   Q4_0 / Q4_1 / Q5_0 / Q5_1  quant plane: 16 B per block (qs, file nibble order)
//          side plane, one record per row of nbr = cols/32 blocks: d[nbr] f16, then m[nbr] f16
//          (Q4_1, Q5_1), then, from the next 4-byte boundary, qh[nbr] u32 (Q5_0, Q5_1; bit j =
//          weight j's fifth bit) -- side_geom(). For the other formats the side plane is the
//          scale plane alone (d per block, block order).
struct WLayout {
    uint64_t quant_bytes;  // bytes of the quant plane (or of the whole Q4_K matrix)
    uint64_t scale_off;    // offset of the scale plane
    uint64_t total;
    uint32_t qblock;       // bytes per block in the quant plane
};

inline WLayout weight_layout(int t, uint32_t rows, uint32_t cols) {
    WLayout L{};
    uint64_t nb = uint64_t(rows) * (cols / block_elems(t));
    switch (t) {
    case HKHIP_Q4_K: L.qblock = 144; break;
    case HKHIP_Q8_0: L.qblock = 32; break;
    case HKHIP_IQ4_NL: case HKHIP_Q4_0: case HKHIP_Q4_1: case HKHIP_Q5_0: case HKHIP_Q5_1: L.qblock = 16; break;
    case HKHIP_Q6_K: L.qblock = 208; break;
    case HKHIP_Q5_K: L.qblock = 176; break;
    case HKHIP_IQ4_XS: L.qblock = 128; break;
    }
    if (fallback_type(t)) L.qblock = uint32_t(block_bytes(t)); // file layout, no planes
    L.quant_bytes = nb * L.qblock;
    if (t == HKHIP_Q4_K || t == HKHIP_Q5_K || fallback_type(t)) {
        L.scale_off = L.quant_bytes;
        L.total = L.quant_bytes;
    } else {
        L.scale_off = align256(L.quant_bytes);
        const uint64_t side = block_elems(t) == 32 ? uint64_t(rows) * side_geom(t, cols / 32).stride
                            : nb * (t == HKHIP_IQ4_XS ? 8 : 2);
        L.total = align256(L.scale_off + side); // the kernels read the scales as aligned words
    }
    return L;
}

// Activation-quant buffer for n tokens of k values. Both kinds live side by side so one
// input serves the 32-weight formats (A8) and the super-block formats (Q8K) alike:
//   a8_qs [n][k] i8, a8_d [n][k/32] f32, a8_s [n][k/32] i32, a8_ds [n][k/32] f32 = d * (f32)s
//         (the offset operand of Q4_1 / Q5_1, as kernelLegacy forms it, gemm.zig:165),
//   a8_dsb [k/256][n][3][8] bf16: a8_ds of the 8 blocks of each super-block as three bf16
//         parts (hi + mid + lo = the f32 value exactly), super-block major so that a token
//         range of one super-block is contiguous -- the token-side operand of the Q4_1 / Q5_1
//         GEMM's offset term, which runs on bf16 MFMAs,
//   k_qs  [n][k] i8, k_d  [n][k/256] f32, k_bs [n][k/16] i16,
//   k_db  [n][k/32] f32: d * (f32)(bsum of the 32 values of each sub-block), the Q5_K GEMM's
//         min-term operand,
//   k_mb  [n][k/256][16] bf16: per super-block, its 8 sub-blocks' 32-value sums as exact bf16
//         integers, bsum32 = 64*u + v with v in [0, 63]: 64*u for the 8 sub-blocks, then v --
//         the token-side operand of the GEMM's integer min term, precomputed once
//   For at most SK_MAX_TOKENS tokens, token-interleaved copies of the Q8K planes for the
//   small-batch kernel, tokens in tiles of 16 (the last tile's padding positions are left
//   unwritten; the kernel's padding lanes read the last token's entries instead):
//   k_il   [k/64][tiles][64][16 B]: entry 16g + p holds token 16*tile + p's values
//          64c + 16g .. 64c + 16g + 15 -- one 16-token tile's 64-value chunk is 1 KB in the
//          order of the MFMA lanes that use it
//   k_ilmb [k/256][tiles][2][16][16 B]: k_mb's two 16-byte halves, token-interleaved
//   k_ild  [k/256][tiles][16] f32: k_d, token-interleaved
constexpr uint32_t SK_MAX_TOKENS = 32;
constexpr uint32_t SK_MIN_TOKENS = 4; // below, the decode kernels are faster
struct ActLayout {
    uint64_t a8_qs, a8_d, a8_s, a8_ds, a8_dsb, k_qs, k_d, k_bs, k_db, k_mb, k_il, k_ilmb, k_ild, total;
    uint32_t tiles; // 16-token tiles of the interleaved planes (0: none)
};

inline ActLayout act_layout(uint32_t n, uint32_t k) {
    ActLayout L{};
    uint64_t nk = uint64_t(n) * k;
    uint64_t o = 0;
    L.a8_qs = o; o = align256(o + nk);
    L.a8_d = o;  o = align256(o + nk / 32 * 4);
    L.a8_s = o;  o = align256(o + nk / 32 * 4);
    L.a8_ds = o; o = align256(o + nk / 32 * 4);
    L.a8_dsb = o; o = align256(o + (k % QK_K == 0 ? nk / QK_K * 48 : 0));
    L.k_qs = o;  o = align256(o + (k % QK_K == 0 ? nk : 0));
    L.k_d = o;   o = align256(o + (k % QK_K == 0 ? nk / QK_K * 4 : 0));
    L.k_bs = o;  o = align256(o + (k % QK_K == 0 ? nk / 16 * 2 : 0));
    L.k_db = o;  o = align256(o + (k % QK_K == 0 ? nk / 32 * 4 : 0));
    L.k_mb = o;  o = align256(o + (k % QK_K == 0 ? nk / QK_K * 32 : 0));
    L.tiles = (k % QK_K == 0 && n >= 1 && n <= SK_MAX_TOKENS) ? (n + 15) / 16 : 0;
    const uint64_t tk = uint64_t(L.tiles) * 16 * k; // interleaved entries (padded tokens)
    L.k_il = o;   o = align256(o + tk);
    L.k_ilmb = o; o = align256(o + tk / QK_K * 32);
    L.k_ild = o;  o = align256(o + tk / QK_K * 4);
    L.total = o;
    return L;
}

struct ActA8 {
    const int8_t *qs;
    const float *d;
};
struct ActQ8K {
    const int8_t *qs;
    const float *d;
    const int16_t *bs;
};

// ---- device helpers ----

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// hk's IQ4_NL codebook (src/quant/tables.zig:13), packed four entries per word, entry 0 in
// the lowest byte, for byte-permute lookups.
constexpr int8_t kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
constexpr uint32_t iq4nl_word(int w) {
    return uint32_t(uint8_t(kvalues_iq4nl[4 * w])) | (uint32_t(uint8_t(kvalues_iq4nl[4 * w + 1])) << 8) |
           (uint32_t(uint8_t(kvalues_iq4nl[4 * w + 2])) << 16) | (uint32_t(uint8_t(kvalues_iq4nl[4 * w + 3])) << 24);
}
constexpr uint32_t IQ4NL_T0 = iq4nl_word(0), IQ4NL_T1 = iq4nl_word(1), IQ4NL_T2 = iq4nl_word(2),
                   IQ4NL_T3 = iq4nl_word(3);
static_assert(IQ4NL_T0 == 0xBFAD9881u && IQ4NL_T3 == 0x71594535u, "codebook packing");

// Four 4-bit indices (one per byte, each < 16) to four signed codebook bytes.
__device__ __forceinline__ uint32_t iq4nl_lookup4(uint32_t idx) {
    uint32_t sel = idx & 0x07070707u;
    uint32_t lo = __builtin_amdgcn_perm(IQ4NL_T1, IQ4NL_T0, sel);
    uint32_t hi = __builtin_amdgcn_perm(IQ4NL_T3, IQ4NL_T2, sel);
    uint32_t m = ((idx >> 3) & 0x01010101u) * 0xFFu; // 0xFF in bytes whose index is >= 8
    return (hi & m) | (lo & ~m);
}

// Four unsigned quants (one per byte, each < 128) minus a zero point z4 = z * 0x01010101 (z <
// 128), as two's-complement bytes: the 0x80 bias keeps the byte subtractions from borrowing.
__device__ __forceinline__ uint32_t sub_zp4(uint32_t u, uint32_t z4) { return ((u | 0x80808080u) - z4) ^ 0x80808080u; }
// Bits 0-3 of b to bit 4 of bytes 0-3 (the shifted copies of b do not overlap: no carries).
__device__ __forceinline__ uint32_t bits_to_b4(uint32_t b) { return ((b & 0xFu) * 0x02040810u) & 0x10101010u; }

// Signed int8 weights of a 32-weight 4/5-bit block, four per word: word i of half hh (hh = 0
// the low nibbles of the block's 16 bytes, weights 4i..4i+3; hh = 1 the high nibbles, weights
// 16 + 4i..), from the block's quant word x (bytes 4i..4i+3) and fifth-bit word qh. Q4_1 and
// Q5_1 stay unsigned (their offset is a separate term); IQ4_NL goes through the codebook.
template <int T> __device__ __forceinline__ uint32_t low_bit_word(uint32_t x, uint32_t qh, uint32_t hh, uint32_t i) {
    uint32_t n = (x >> (4 * hh)) & 0x0F0F0F0Fu;
    if constexpr (T == HKHIP_IQ4_NL) return iq4nl_lookup4(n);
    if constexpr (has_qh(T)) n |= bits_to_b4(qh >> (16 * hh + 4 * i));
    if constexpr (zero_point(T) != 0) n = sub_zp4(n, uint32_t(zero_point(T)) * 0x01010101u);
    return n;
}

// 16 (4) bytes per lane global -> LDS: lane L writes at the wave-uniform LDS address + 16*L
// (4*L). Issued as inline assembly: the compiler then keeps no books on these loads (the kernels
// wait for them with explicit counts), where for the builtin it would wait for all of them before
// an LDS read it cannot prove independent -- which drains the prefetch ring every step.
__device__ __forceinline__ uint32_t lds_addr(const void *lds) {
    return uint32_t((uintptr_t)(const __attribute__((address_space(3))) void *)lds);
}
__device__ __forceinline__ void load_lds16(const void *g, void *lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(lds_addr(lds)) : "memory", "m0");
}
__device__ __forceinline__ void load_lds4(const void *g, void *lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" : : "v"(g), "s"(lds_addr(lds)) : "memory", "m0");
}

// Output mode HKHIP_SILU_MUL: output i of gate g (row 2i) and up u (row 2i + 1), as
// shaders/mmvq.comp:186 computes it.
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// ---- launchers (defined in the kernel files) ----

hipError_t launch_repack(int t, const uint8_t *src, uint8_t *dst, uint32_t rows, uint32_t cols, hipStream_t s);
hipError_t launch_dequant(int t, const uint8_t *w, uint32_t rows, uint32_t cols, uint32_t row0, uint32_t nrows,
                          float *out, hipStream_t s);
// Rows ids[0..n) (device array; each below rows) decoded to out [n][cols] (embedding lookup).
hipError_t launch_dequant_gather(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint32_t *ids, uint32_t n,
                                 float *out, hipStream_t s);

// fallback.hip: the float-decode formats (fallback_type): bit-exact decode of rows (or of rows
// ids[] when ids is not null) and the decode-based products for 1..8 tokens of an f32 input (x)
// or of a prepared activation buffer (xq; not NVFP4, whose products take f32 inputs).
hipError_t launch_fb_dequant(int t, const uint8_t *w, uint32_t cols, uint32_t row0, const uint32_t *ids, uint32_t nrows,
                             float *out, hipStream_t s);
struct MvPartDesc;
hipError_t launch_fb_mv(int t, const MvPartDesc *parts, int nparts, uint32_t K, const float *x, const uint8_t *xq,
                        uint32_t n, int mode, hipStream_t s);
hipError_t launch_qact(const float *x, uint32_t n, uint32_t k, int kind, uint8_t *xq, hipStream_t s);
// qact with the RMS norm (weights `norm`, or null for none) folded in, by token rows.
hipError_t launch_qact_row(const float *x, uint32_t n, uint32_t k, int kind, uint8_t *xq, const float *norm, float eps,
                           hipStream_t s);
hipError_t launch_act_pack(const uint8_t *xq, uint32_t n, uint32_t k, int kind, uint8_t *out, hipStream_t s);
// One matrix of a fused decode launch (all parts share cols and the input).
struct MvPartDesc {
    const uint8_t *w;
    float *y;
    const float *bias;
    uint32_t rows;
};
hipError_t launch_mmvq_parts(int t, const MvPartDesc *parts, int nparts, uint32_t K, const float *x,
                             const uint8_t *xq, uint32_t n, int mode, hipStream_t s);
// The same with the f32 input RMS-normalized per token first (norm weights [cols], eps), fused into
// the kernel's staging; hipErrorNotSupported when the chosen kernel cannot fuse it (the caller then
// normalizes separately).
hipError_t launch_mmvq_parts_norm(int t, const MvPartDesc *parts, int nparts, uint32_t K, const float *x,
                                  const uint8_t *xq, uint32_t n, int mode, const float *norm, float eps,
                                  hipStream_t s);
hipError_t launch_mmvq(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n,
                       float *y, const float *bias, int mode, hipStream_t s);
bool mm2_supports(int t, uint32_t rows, uint32_t cols, uint32_t n);
// Small-batch MFMA product (Q4_K, 1..32 tokens): weights streamed like the decode kernels.
bool mmsk_supports(int t, uint32_t rows, uint32_t cols, uint32_t n);
hipError_t launch_mmsk(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n,
                       float *y, const float *bias, int mode, hipStream_t s);
hipError_t launch_mmsk_parts(int t, const MvPartDesc *parts, int nparts, uint32_t cols, const uint8_t *xq,
                             uint32_t n, int mode, hipStream_t s);
// Prefill GEMM for Q6_K, Q8_0 and IQ4_NL (cols a multiple of 256).
bool mmx_supports(int t, uint32_t rows, uint32_t cols, uint32_t n);
hipError_t launch_mmx(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n, float *y,
                      const float *bias, int mode, hipStream_t s);
hipError_t launch_mm2(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n, float *y,
                      const float *bias, int mode, hipStream_t s);
hipError_t launch_mm(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n,
                     float *y, const float *bias, int mode, hipStream_t s);


// Q6_K int8 operand planes. Four weights q (bytes in [0, 63]) of one 16-weight group with the
// signed group scale sc: w = sc*(q - 32) lies in [-4096, 4096]. In 16-bit lanes (the even and the
// odd bytes of the word spread by one byte permute each, then one packed multiply-add each with
// m = 4*sc and k = 128 - 128*sc in both halves) y = 4*w + 128 lies in [-16256, 16512]; its high
// byte H = floor(y / 256) lies in [-64, 64] and its low byte minus 128, L, in [-128, 127], so that
// 4*w = 256*H + L exactly: H is the high bytes of the four lanes and L their low bytes with the top
// bit flipped, one byte permute each. (The same planes as x = w + 32, H = x >> 6, L = 4*((x & 63)
// - 32), with six VALU instructions per word fewer.)
__device__ __forceinline__ void q6k_planes(uint32_t q, uint32_t m, uint32_t k, int &H, int &L) {
    typedef unsigned short u2 __attribute__((ext_vector_type(2)));
    const u2 mm = __builtin_bit_cast(u2, m), kk = __builtin_bit_cast(u2, k);
    const u2 ye = __builtin_bit_cast(u2, __builtin_amdgcn_perm(0u, q, 0x0C020C00u)) * mm + kk; // bytes 0, 2
    const u2 yo = __builtin_bit_cast(u2, __builtin_amdgcn_perm(0u, q, 0x0C030C01u)) * mm + kk; // bytes 1, 3
    const uint32_t e = __builtin_bit_cast(uint32_t, ye), o = __builtin_bit_cast(uint32_t, yo);
    H = int(__builtin_amdgcn_perm(o, e, 0x07030501u));
    L = int(__builtin_amdgcn_perm(o, e, 0x06020400u) ^ 0x80808080u);
}
// q6k_planes' factors for the group scale sc.
__device__ __forceinline__ uint32_t q6k_m(int sc) { return (uint32_t(4 * sc) & 0xFFFFu) * 0x00010001u; }
__device__ __forceinline__ uint32_t q6k_k(int sc) { return (uint32_t(128 - 128 * sc) & 0xFFFFu) * 0x00010001u; }

} // namespace hkhip
