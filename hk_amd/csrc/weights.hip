// Weight upload repack (file layout -> device layout) and the bit-exact dequantizer.
//
// The decoders restate src/quant/dequant.zig (q4_0 24-31, q4_1 33-41, q5_0 43-56, q5_1 58-72,
// q8_0 74-78, scaleMinK4 166-175, q4_k 177-202, q5_k 204-235, q6_k 237-267, iq4_nl 430-437,
// iq4_xs 439-455). The library is
// built with -ffp-contract=off, so every multiply and add below rounds separately, as in the Zig
// source, and the f32 results are bit-identical to hk's CPU decoders.
#include "common.hpp"

namespace hkhip {

// Side-plane addresses of block b (row b / nbr, column block b % nbr) of a 4/5-bit format.
struct SideRef {
    uint64_t d, m, qh; // byte offsets from the side plane
};
__host__ __device__ inline SideRef side_ref(int t, uint64_t b, uint32_t nbr) {
    const SideGeom G = side_geom(t, nbr);
    const uint64_t r = b / nbr, c = b % nbr, base = r * G.stride;
    return SideRef{base + 2 * c, base + G.m_off + 2 * c, base + G.qh_off + 4 * c};
}

// One thread per block: file block b -> quant plane block b (16-byte aligned) + its side-plane
// entries.
__global__ void repack_kernel(int t, const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, uint64_t nblocks,
                              uint64_t scale_off, uint32_t nbr) {
    uint64_t b = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    uint16_t *scales = reinterpret_cast<uint16_t *>(dst + scale_off);
    if (t == HKHIP_Q4_0 || t == HKHIP_Q4_1 || t == HKHIP_Q5_0 || t == HKHIP_Q5_1) {
        // blocks.zig:13-16: d, [m], [qh[4]], qs[16]
        const uint8_t *s = src + b * block_bytes_dev(t);
        uint8_t *side = dst + scale_off;
        const SideRef R = side_ref(t, b, nbr);
        side[R.d] = s[0];
        side[R.d + 1] = s[1];
        uint32_t o = 2;
        if (has_m(t)) {
            side[R.m] = s[2];
            side[R.m + 1] = s[3];
            o = 4;
        }
        if (has_qh(t)) {
            for (int k = 0; k < 4; k++) side[R.qh + k] = s[o + k];
            o += 4;
        }
        uint8_t *q = dst + b * 16;
        for (int j = 0; j < 16; j++) q[j] = s[o + j];
    } else if (t == HKHIP_IQ4_XS) { // blocks.zig:35: d, scales_h, scales_l[4] | qs[128]
        const uint8_t *s = src + b * 136;
        uint8_t *hdr = dst + scale_off + b * 8;
        for (int j = 0; j < 8; j++) hdr[j] = s[j];
        uint8_t *q = dst + b * 128;
        for (int j = 0; j < 128; j++) q[j] = s[8 + j];
    } else if (t == HKHIP_Q8_0) {
        const uint8_t *s = src + b * 34;
        scales[b] = uint16_t(s[0] | (s[1] << 8));
        uint8_t *q = dst + b * 32;
        for (int j = 0; j < 32; j++) q[j] = s[2 + j];
    } else if (t == HKHIP_IQ4_NL) {
        const uint8_t *s = src + b * 18;
        scales[b] = uint16_t(s[0] | (s[1] << 8));
        uint8_t *q = dst + b * 16;
        for (int j = 0; j < 16; j++) q[j] = s[2 + j];
    } else { // Q6_K: ql[128] qh[64] scales[16] d
        const uint8_t *s = src + b * 210;
        scales[b] = uint16_t(s[208] | (s[209] << 8));
        uint8_t *q = dst + b * 208;
        for (int j = 0; j < 208; j++) q[j] = s[j];
    }
}

hipError_t launch_repack(int t, const uint8_t *src, uint8_t *dst, uint32_t rows, uint32_t cols, hipStream_t s) {
    WLayout L = weight_layout(t, rows, cols);
    uint64_t nb = uint64_t(rows) * (cols / block_elems(t));
    if (t == HKHIP_Q4_K || t == HKHIP_Q5_K) return hipMemcpyAsync(dst, src, L.total, hipMemcpyDeviceToDevice, s);
    if (nb == 0) return hipSuccess;
    uint32_t grid = uint32_t((nb + 255) / 256);
    repack_kernel<<<grid, 256, 0, s>>>(t, src, dst, nb, L.scale_off, cols / 32);
    return hipGetLastError();
}

// dequant.zig:166-175 scaleMinK4
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *q, uint32_t &sc, uint32_t &mn) {
    if (j < 4) {
        sc = q[j] & 63;
        mn = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// One thread per output weight of rows [row0, row0 + nrows). Out is [nrows][cols].
__global__ void dequant_kernel(int t, const uint8_t *__restrict__ w, uint32_t cols, uint32_t row0, uint64_t total,
                               uint64_t scale_off, float *__restrict__ out, const uint32_t *__restrict__ ids) {
    uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= total) return;
    uint64_t r = ids ? uint64_t(ids[i / cols]) : row0 + i / cols; // gather: output row j is row ids[j]
    uint32_t c = uint32_t(i % cols);
    const uint16_t *scales = reinterpret_cast<const uint16_t *>(w + scale_off);
    float v;
    if (t == HKHIP_Q4_0 || t == HKHIP_Q4_1 || t == HKHIP_Q5_0 || t == HKHIP_Q5_1) {
        const uint64_t b = r * (cols / 32) + c / 32;
        const uint8_t *side = w + scale_off;
        const SideRef R = side_ref(t, b, cols / 32);
        const float d = f16_bits_to_f32(side[R.d] | (side[R.d + 1] << 8));
        const uint32_t j = c % 32;
        const uint8_t byte = w[b * 16 + (j & 15)];
        uint32_t u = j < 16 ? (byte & 0x0F) : (byte >> 4);
        if (has_qh(t)) {
            const uint32_t qh = side[R.qh] | (side[R.qh + 1] << 8) | (side[R.qh + 2] << 16) | (uint32_t(side[R.qh + 3]) << 24);
            u |= ((qh >> j) & 1u) << 4;
        }
        if (has_m(t))
            v = (float)u * d + f16_bits_to_f32(side[R.m] | (side[R.m + 1] << 8));
        else
            v = (float)(int(u) - zero_point(t)) * d;
    } else if (t == HKHIP_Q8_0) {
        uint64_t b = r * (cols / 32) + c / 32;
        float d = f16_bits_to_f32(scales[b]);
        v = (float)(int8_t)w[b * 32 + (c % 32)] * d;
    } else if (t == HKHIP_IQ4_NL) {
        uint64_t b = r * (cols / 32) + c / 32;
        float d = f16_bits_to_f32(scales[b]);
        uint32_t j = c % 32;
        uint8_t byte = w[b * 16 + (j & 15)];
        uint32_t idx = j < 16 ? (byte & 0x0F) : (byte >> 4);
        int8_t q = (int8_t)(iq4nl_lookup4(idx) & 0xFF);
        v = d * (float)q;
    } else if (t == HKHIP_IQ4_XS) { // dequant.zig:439-455
        const uint64_t b = r * (cols / 256) + c / 256;
        const uint8_t *hdr = w + scale_off + b * 8;
        const uint32_t j = c % 256, ib = j / 32, l = j % 32;
        const uint32_t scales_h = hdr[2] | (hdr[3] << 8);
        const uint32_t lo = (hdr[4 + ib / 2] >> (4 * (ib % 2))) & 0x0F, hi = (scales_h >> (2 * ib)) & 3;
        const float dl = f16_bits_to_f32(hdr[0] | (hdr[1] << 8)) * (float)(int(lo | (hi << 4)) - 32);
        const uint8_t byte = w[b * 128 + 16 * ib + (l & 15)];
        const int8_t q = (int8_t)(iq4nl_lookup4(l < 16 ? (byte & 0x0F) : (byte >> 4)) & 0xFF);
        v = dl * (float)q;
    } else if (t == HKHIP_Q4_K || t == HKHIP_Q5_K) { // Q5_K: dequant.zig:204-235
        const bool five = t == HKHIP_Q5_K;
        uint64_t b = r * (cols / 256) + c / 256;
        const uint8_t *blk = w + b * (five ? 176 : 144);
        float d = f16_bits_to_f32(blk[0] | (blk[1] << 8));
        float dmin = f16_bits_to_f32(blk[2] | (blk[3] << 8));
        uint32_t j = c % 256;
        uint32_t chunk = j / 64, hi = (j % 64) / 32, l = j % 32;
        uint32_t sc, mn;
        scale_min_k4(int(2 * chunk + hi), blk + 4, sc, mn);
        float d1 = d * (float)sc;
        float m1 = dmin * (float)mn;
        uint8_t q = blk[(five ? 48 : 16) + 32 * chunk + l];
        uint32_t nib = hi ? (q >> 4) : (q & 0x0F);
        if (five) nib += ((blk[16 + l] >> (2 * chunk + hi)) & 1) * 16;
        v = d1 * (float)nib - m1;
    } else { // Q6_K
        uint64_t b = r * (cols / 256) + c / 256;
        const uint8_t *blk = w + b * 208;
        float d = f16_bits_to_f32(scales[b]);
        uint32_t j = c % 256;
        uint32_t n = j / 128, part = (j % 128) / 32, l = j % 32;
        const uint8_t *ql = blk + 64 * n, *qh = blk + 128 + 32 * n;
        const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192) + 8 * n;
        uint32_t lo = (part & 1) ? ql[l + 32] : ql[l];
        uint32_t low4 = (part & 2) ? (lo >> 4) : (lo & 0x0F);
        uint32_t h2 = (qh[l] >> (2 * part)) & 3;
        int q = int(low4 | (h2 << 4)) - 32;
        v = d * (float)(int(sc[l / 16 + 2 * part]) * q);
    }
    out[i] = v;
}

hipError_t launch_dequant(int t, const uint8_t *w, uint32_t rows, uint32_t cols, uint32_t row0, uint32_t nrows,
                          float *out, hipStream_t s) {
    if (fallback_type(t)) return launch_fb_dequant(t, w, cols, row0, nullptr, nrows, out, s);
    WLayout L = weight_layout(t, rows, cols);
    uint64_t total = uint64_t(nrows) * cols;
    if (total == 0) return hipSuccess;
    uint64_t grid = (total + 255) / 256;
    if (grid > 0x7fffffffu) return hipErrorInvalidValue;
    dequant_kernel<<<uint32_t(grid), 256, 0, s>>>(t, w, cols, row0, total, L.scale_off, out, nullptr);
    return hipGetLastError();
}

hipError_t launch_dequant_gather(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint32_t *ids, uint32_t n,
                                 float *out, hipStream_t s) {
    if (fallback_type(t)) return launch_fb_dequant(t, w, cols, 0, ids, n, out, s);
    WLayout L = weight_layout(t, rows, cols);
    uint64_t total = uint64_t(n) * cols;
    if (total == 0) return hipSuccess;
    uint64_t grid = (total + 255) / 256;
    if (grid > 0x7fffffffu) return hipErrorInvalidValue;
    dequant_kernel<<<uint32_t(grid), 256, 0, s>>>(t, w, cols, 0, total, L.scale_off, out, ids);
    return hipGetLastError();
}

} // namespace hkhip
