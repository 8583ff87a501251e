/* CPU oracle for hk's quantized-linear hot path. TEST INFRASTRUCTURE ONLY.
 *
 * Restates, in plain C, the arithmetic of the reference CPU kernels:
 *   - block decoders           src/quant/dequant.zig:24-78, 166-202, 237-267, 430-437, 550-591
 *   - activation quantizers    src/quant/vecdot.zig:134-180
 *   - single-row dots          src/quant/vecdot.zig:235-384, 459-570, 725-771
 *   - register-tiled GEMM      src/quant/gemm.zig:131-236, 262-313, 504-520
 *   - canonical unpack         src/quant/unpack.zig:29-76, 81-160
 *   - matmul dispatch          src/engine/matmul.zig:18, 96-153 (n >= 8 -> tiles)
 *
 * Integer parts are exact. Float parts follow the reference's operation order,
 * including its eight-lane accumulators (isa.zig:57-60 lane definition of the
 * dot-4 primitive), @mulAdd as fmaf and @reduce(.Add) as an in-order lane sum.
 * Build with -ffp-contract=off so that no other multiply-add is fused.
 *
 * Pins (what checks each part): tests/test_oracle.py holds them; the decoders
 * are checked bit-for-bit against the reference's gguf-generated fixtures, the
 * quantizers against their closed forms and invariants, the dots against an
 * independent float64 decode-dot and an independent exact-integer restatement,
 * and the tiled GEMM against the row dots.
 */
#include "hk_oracle.h"

#include <math.h>
#include <string.h>

#define QK_K 256

static const int8_t kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                         1,    13,   25,  38,  53,  69,  89,  113};
/* tables.zig:13 */

float hko_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff, bits;
    float f;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            f = ldexpf((float)m, -24); /* exact: m < 2^10 */
            return sign ? -f : f;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline float h16(const uint8_t *p) { return hko_f16_to_f32(rd16(p)); }

int hko_block_elems(int t) {
    switch (t) {
    case HKO_Q8_0: case HKO_IQ4_NL: case HKO_Q4_0: case HKO_Q4_1: case HKO_Q5_0: case HKO_Q5_1: return 32;
    case HKO_Q4_K: case HKO_Q5_K: case HKO_Q6_K: case HKO_IQ4_XS: return QK_K;
    default: return hko_fb_block_elems(t);
    }
}

int hko_block_bytes(int t) {
    switch (t) {
    case HKO_Q8_0: return 34;   /* blocks.zig:17 */
    case HKO_IQ4_NL: return 18; /* blocks.zig:34 */
    case HKO_Q4_K: return 144;  /* blocks.zig:21 */
    case HKO_Q6_K: return 210;  /* blocks.zig:23 */
    case HKO_Q5_K: return 176;  /* blocks.zig:22 */
    case HKO_IQ4_XS: return 136; /* blocks.zig:35 */
    case HKO_Q4_0: return 18;   /* blocks.zig:13 */
    case HKO_Q4_1: return 20;   /* blocks.zig:14 */
    case HKO_Q5_0: return 22;   /* blocks.zig:15 */
    case HKO_Q5_1: return 24;   /* blocks.zig:16 */
    default: return hko_fb_block_bytes(t);
    }
}

int hko_act_kind(int t) {
    switch (t) {
    case HKO_Q8_0: case HKO_IQ4_NL: case HKO_Q4_0: case HKO_Q4_1: case HKO_Q5_0: case HKO_Q5_1:
        return 0; /* vecdot.zig:187 */
    case HKO_Q4_K: case HKO_Q5_K: case HKO_Q6_K: case HKO_IQ4_XS: return 1; /* vecdot.zig:188 */
    default: return hko_fb_act_kind(t);
    }
}

/* ---------------------------------------------------------------------------------------------
 * Decoders (dequant.zig)
 * ------------------------------------------------------------------------------------------- */

/* dequant.zig:166-175 */
void hko_scale_min_k4(int j, const uint8_t q[12], uint8_t *sc, uint8_t *mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* vecdot.zig:461-474: the same unpack done on 32-bit words. */
void hko_scales_mins_k4_words(const uint8_t p[12], uint8_t sc[8], uint8_t mn[8]) {
    const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
    uint32_t u[4];
    for (int i = 0; i < 3; i++)
        u[i] = (uint32_t)p[4 * i] | ((uint32_t)p[4 * i + 1] << 8) | ((uint32_t)p[4 * i + 2] << 16) |
               ((uint32_t)p[4 * i + 3] << 24);
    u[3] = ((u[2] >> 4) & k2) | (((u[1] >> 6) & k3) << 4);
    uint32_t aux = u[1] & k1;
    u[1] = (u[2] & k2) | (((u[0] >> 6) & k3) << 4);
    u[2] = aux;
    u[0] &= k1;
    for (int i = 0; i < 4; i++) {
        sc[i] = (uint8_t)(u[0] >> (8 * i));
        sc[4 + i] = (uint8_t)(u[1] >> (8 * i));
        mn[i] = (uint8_t)(u[2] >> (8 * i));
        mn[4 + i] = (uint8_t)(u[3] >> (8 * i));
    }
}

/* The unsigned quants of a Q4_0 / Q4_1 / Q5_0 / Q5_1 block, weight order: byte j's low nibble is
 * weight j, its high nibble weight j + 16 (dequant.zig:24-70); Q5 adds bit j of the little-endian
 * qh word as bit 4 of weight j. Returns the block's quant bytes' offset. */
static int low_bit_quants(int t, const uint8_t *b, int32_t u[32]) {
    int qs = (t == HKO_Q4_0) ? 2 : 4;
    uint32_t qh = 0;
    if (t == HKO_Q5_0) { qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24); qs = 6; }
    if (t == HKO_Q5_1) { qh = (uint32_t)b[4] | ((uint32_t)b[5] << 8) | ((uint32_t)b[6] << 16) | ((uint32_t)b[7] << 24); qs = 8; }
    for (int j = 0; j < 16; j++) {
        u[j] = b[qs + j] & 0x0F;
        u[j + 16] = b[qs + j] >> 4;
        if (t == HKO_Q5_0 || t == HKO_Q5_1) {
            u[j] |= (int32_t)(((qh >> j) << 4) & 0x10);
            u[j + 16] |= (int32_t)((qh >> (j + 12)) & 0x10);
        }
    }
    return qs;
}

/* Zero point (gemm.zig:262-270 legacyZeroPoint) and whether a block has an offset m. */
static int low_bit_zp(int t) { return t == HKO_Q4_0 ? 8 : t == HKO_Q5_0 ? 16 : 0; }
static int low_bit_has_m(int t) { return t == HKO_Q4_1 || t == HKO_Q5_1; }

/* dequant.zig:24-70: d * (u - zp), or d * u + m. */
static void deq_low_bit(int t, const uint8_t *b, float *out) {
    int32_t u[32];
    low_bit_quants(t, b, u);
    float d = h16(b);
    if (low_bit_has_m(t)) {
        float m = h16(b + 2);
        for (int j = 0; j < 32; j++) out[j] = (float)u[j] * d + m;
    } else {
        int zp = low_bit_zp(t);
        for (int j = 0; j < 32; j++) out[j] = (float)(u[j] - zp) * d;
    }
}

/* dequant.zig:74-78 */
static void deq_q8_0(const uint8_t *b, float *out) {
    float d = h16(b);
    for (int j = 0; j < 32; j++) out[j] = (float)(int8_t)b[2 + j] * d;
}

/* dequant.zig:177-202 */
static void deq_q4_k(const uint8_t *b, float *out) {
    float d = h16(b), min = h16(b + 2);
    const uint8_t *scales = b + 4, *qs = b + 16;
    int is = 0, o = 0, q = 0;
    for (int j = 0; j < 256; j += 64) {
        uint8_t sc, mn;
        hko_scale_min_k4(is, scales, &sc, &mn);
        float d1 = d * (float)sc, m1 = min * (float)mn;
        hko_scale_min_k4(is + 1, scales, &sc, &mn);
        float d2 = d * (float)sc, m2 = min * (float)mn;
        for (int l = 0; l < 32; l++) {
            out[o + l] = d1 * (float)(qs[q + l] & 0x0F) - m1;
            out[o + 32 + l] = d2 * (float)(qs[q + l] >> 4) - m2;
        }
        o += 64;
        q += 32;
        is += 2;
    }
}

/* dequant.zig:237-267 */
static void deq_q6_k(const uint8_t *b, float *out) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *scales = (const int8_t *)(b + 192);
    float d = h16(b + 208);
    int o = 0, l0 = 0, h0 = 0, s0 = 0;
    for (int n = 0; n < 256; n += 128) {
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int lo0 = ql[l0 + l] & 0x0F, lo1 = ql[l0 + l + 32] & 0x0F;
            int hi0 = ql[l0 + l] >> 4, hi1 = ql[l0 + l + 32] >> 4;
            int h8 = qh[h0 + l];
            int q1 = (lo0 | (((h8 >> 0) & 3) << 4)) - 32;
            int q2 = (lo1 | (((h8 >> 2) & 3) << 4)) - 32;
            int q3 = (hi0 | (((h8 >> 4) & 3) << 4)) - 32;
            int q4 = (hi1 | (((h8 >> 6) & 3) << 4)) - 32;
            out[o + l + 0] = d * (float)(scales[s0 + is + 0] * q1);
            out[o + l + 32] = d * (float)(scales[s0 + is + 2] * q2);
            out[o + l + 64] = d * (float)(scales[s0 + is + 4] * q3);
            out[o + l + 96] = d * (float)(scales[s0 + is + 6] * q4);
        }
        o += 128;
        l0 += 64;
        h0 += 32;
        s0 += 8;
    }
}

/* dequant.zig:204-235: Q4_K's decode with the fifth bit of weight l of chunk c's low (high) half
 * at bit 2c (2c + 1) of qh[l]. */
static void deq_q5_k(const uint8_t *b, float *out) {
    float d = h16(b), min = h16(b + 2);
    const uint8_t *qh = b + 16, *qs = b + 48;
    for (int c = 0; c < 4; c++) {
        uint8_t sc, mn;
        hko_scale_min_k4(2 * c, b + 4, &sc, &mn);
        float d1 = d * (float)sc, m1 = min * (float)mn;
        hko_scale_min_k4(2 * c + 1, b + 4, &sc, &mn);
        float d2 = d * (float)sc, m2 = min * (float)mn;
        for (int l = 0; l < 32; l++) {
            uint32_t lo = (qs[32 * c + l] & 0x0F) + ((qh[l] >> (2 * c)) & 1 ? 16 : 0);
            uint32_t hi = (qs[32 * c + l] >> 4) + ((qh[l] >> (2 * c + 1)) & 1 ? 16 : 0);
            out[64 * c + l] = d1 * (float)lo - m1;
            out[64 * c + 32 + l] = d2 * (float)hi - m2;
        }
    }
}

/* IQ4_XS sub-block scale ls = (6-bit scale) - 32 (dequant.zig:443-447, vecdot.zig:577-582). */
static int32_t iq4xs_ls(const uint8_t *b, int ib) {
    uint32_t scales_h = (uint32_t)b[2] | ((uint32_t)b[3] << 8);
    uint32_t lo = (b[4 + ib / 2] >> (4 * (ib % 2))) & 0x0F, hi = (scales_h >> (2 * ib)) & 3;
    return (int32_t)(lo | (hi << 4)) - 32;
}

/* dequant.zig:439-455 */
static void deq_iq4_xs(const uint8_t *b, float *out) {
    float d = h16(b);
    for (int ib = 0; ib < 8; ib++) {
        float dl = d * (float)iq4xs_ls(b, ib);
        const uint8_t *qs = b + 8 + 16 * ib;
        for (int j = 0; j < 16; j++) {
            out[32 * ib + j] = dl * (float)kvalues_iq4nl[qs[j] & 0x0F];
            out[32 * ib + j + 16] = dl * (float)kvalues_iq4nl[qs[j] >> 4];
        }
    }
}

/* dequant.zig:430-437 */
static void deq_iq4_nl(const uint8_t *b, float *out) {
    float d = h16(b);
    for (int j = 0; j < 16; j++) {
        out[j] = d * (float)kvalues_iq4nl[b[2 + j] & 0x0F];
        out[j + 16] = d * (float)kvalues_iq4nl[b[2 + j] >> 4];
    }
}

/* dequant.zig:550-591 */
int hko_dequantize_row(int t, const uint8_t *src, size_t src_len, float *dst, size_t n) {
    int elems = hko_block_elems(t), bytes = hko_block_bytes(t);
    if (!elems) return -1;
    if (n % (size_t)elems) return -1;
    size_t nb = n / (size_t)elems;
    if (src_len != nb * (size_t)bytes) return -1;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = src + i * bytes;
        float *o = dst + i * elems;
        switch (t) {
        case HKO_Q8_0: deq_q8_0(b, o); break;
        case HKO_Q4_K: deq_q4_k(b, o); break;
        case HKO_Q6_K: deq_q6_k(b, o); break;
        case HKO_IQ4_NL: deq_iq4_nl(b, o); break;
        case HKO_Q5_K: deq_q5_k(b, o); break;
        case HKO_IQ4_XS: deq_iq4_xs(b, o); break;
        case HKO_Q4_0: case HKO_Q4_1: case HKO_Q5_0: case HKO_Q5_1: deq_low_bit(t, b, o); break;
        default: hko_fb_decode_block(t, b, o); break;
        }
    }
    return 0;
}

/* ---------------------------------------------------------------------------------------------
 * Activation quantizers (vecdot.zig:134-180). Zig's @round rounds half away from zero, as roundf.
 * ------------------------------------------------------------------------------------------- */

void hko_quantize_a8(const float *x, size_t n, hko_block_a8 *out) {
    for (size_t b = 0; b < n / 32; b++) {
        const float *v = x + b * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            float a = fabsf(v[j]);
            if (a > amax) amax = a; /* @reduce(.Max) over finite values */
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        int32_t s = 0;
        for (int j = 0; j < 32; j++) {
            int32_t q = (int32_t)roundf(v[j] * id);
            out[b].qs[j] = (int8_t)q;
            s += q;
        }
        out[b].d = d;
        out[b].s = s;
    }
}

void hko_quantize_q8k(const float *x, size_t n, hko_block_q8k *out) {
    for (size_t b = 0; b < n / QK_K; b++) {
        const float *src = x + b * QK_K;
        hko_block_q8k *o = out + b;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < QK_K; j++) {
            float a = fabsf(src[j]);
            if (a > amax) {
                amax = a;
                max = src[j];
            }
        }
        if (amax == 0.0f) {
            memset(o, 0, sizeof(*o));
            continue;
        }
        float iscale = -127.0f / max;
        for (int j = 0; j < QK_K; j++) {
            int32_t v = (int32_t)roundf(iscale * src[j]);
            o->qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; j++) {
            int32_t s = 0;
            for (int k = 0; k < 16; k++) s += o->qs[j * 16 + k];
            o->bsums[j] = (int16_t)s;
        }
        o->d = 1.0f / iscale;
    }
}

/* ---------------------------------------------------------------------------------------------
 * Row dots (vecdot.zig). Lane L of the eight-lane accumulators holds, for each 32-byte chunk,
 * the products of bytes 4L..4L+3 (isa.zig:57-60 dpu / dps definition).
 * ------------------------------------------------------------------------------------------- */

/* dpu/dps over one 32-byte chunk: lane L sums a[4L+k] * b[4L+k], k < 4. */
static inline void dp32(int32_t lane[8], const int32_t a[32], const int8_t *b) {
    for (int L = 0; L < 8; L++)
        lane[L] = a[4 * L] * b[4 * L] + a[4 * L + 1] * b[4 * L + 1] + a[4 * L + 2] * b[4 * L + 2] +
                  a[4 * L + 3] * b[4 * L + 3];
}

static inline float reduce8(const float v[8]) {
    float s = v[0];
    for (int L = 1; L < 8; L++) s += v[L];
    return s;
}

/* vecdot.zig:235-250 (Q8_0) and 369-384 (IQ4_NL): signed weights against A8. */
static float dot_legacy(int t, const uint8_t *row, size_t nb, const hko_block_a8 *a) {
    float accf[8] = {0};
    int32_t w[32], di[8];
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = row + i * (size_t)hko_block_bytes(t);
        if (t == HKO_Q8_0) {
            for (int j = 0; j < 32; j++) w[j] = (int8_t)b[2 + j];
        } else {
            for (int j = 0; j < 16; j++) {
                w[j] = kvalues_iq4nl[b[2 + j] & 0x0F]; /* nibbles(): low nibbles first */
                w[j + 16] = kvalues_iq4nl[b[2 + j] >> 4];
            }
        }
        float dv = h16(b);
        float s = dv * a[i].d;
        dp32(di, w, a[i].qs);
        for (int L = 0; L < 8; L++) accf[L] = fmaf((float)di[L], s, accf[L]);
    }
    return reduce8(accf);
}

/* vecdot.zig:293-367 (dotQ4_0, dotQ4_1, dotQ5_0, dotQ5_1): unsigned quants against A8. The zero
 * point comes off lane 0 only (lane0(zp * s)); the offset term m * (d_a * s) is added to every
 * lane, so the eight lanes' sum is scaled back by 1/8. */
static float dot_low_bit(int t, const uint8_t *row, size_t nb, const hko_block_a8 *a) {
    float accf[8] = {0}, extra[8] = {0};
    int32_t u[32], di[8];
    const int zp = low_bit_zp(t), has_m = low_bit_has_m(t);
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = row + i * (size_t)hko_block_bytes(t);
        low_bit_quants(t, b, u);
        float dv = h16(b);
        dp32(di, u, a[i].qs);
        di[0] -= zp * a[i].s;
        float s = dv * a[i].d;
        for (int L = 0; L < 8; L++) accf[L] = fmaf((float)di[L], s, accf[L]);
        if (has_m) {
            float mv = h16(b + 2), ds = a[i].d * (float)a[i].s;
            for (int L = 0; L < 8; L++) extra[L] = fmaf(mv, ds, extra[L]);
        }
    }
    return has_m ? reduce8(accf) + reduce8(extra) * (1.0f / 8.0f) : reduce8(accf);
}

/* vecdot.zig:482-522 k4Block / dotQ4K */
static float dot_q4_k(int t, const uint8_t *row, size_t nsb, const hko_block_q8k *a) {
    float accf[8] = {0}, corr[8] = {0};
    int32_t lo[32], hi[32], t0[8], t1[8];
    const int five = t == HKO_Q5_K, qoff = five ? 48 : 16;
    for (size_t i = 0; i < nsb; i++) {
        const uint8_t *b = row + i * (size_t)hko_block_bytes(t);
        uint8_t sc[8], mn[8];
        hko_scales_mins_k4_words(b + 4, sc, mn);
        int32_t acci[8] = {0};
        for (int p = 0; p < 4; p++) {
            const uint8_t *q = b + qoff + 32 * p;
            for (int j = 0; j < 32; j++) {
                lo[j] = q[j] & 0x0F;
                hi[j] = q[j] >> 4;
                if (five) { /* k4Block has_high (vecdot.zig:492-495) */
                    lo[j] |= ((b[16 + j] >> (2 * p)) & 1) << 4;
                    hi[j] |= ((b[16 + j] >> (2 * p + 1)) & 1) << 4;
                }
            }
            dp32(t0, lo, a[i].qs + p * 64);
            dp32(t1, hi, a[i].qs + p * 64 + 32);
            for (int L = 0; L < 8; L++) acci[L] += t0[L] * sc[2 * p] + t1[L] * sc[2 * p + 1];
        }
        float d = h16(b), dm = h16(b + 2);
        float sd = d * a[i].d, sm = dm * a[i].d;
        for (int L = 0; L < 8; L++) {
            int32_t cs = a[i].bsums[2 * L] * mn[L] + a[i].bsums[2 * L + 1] * mn[L];
            accf[L] = fmaf((float)acci[L], sd, accf[L]);
            corr[L] = fmaf((float)cs, sm, corr[L]);
        }
    }
    return reduce8(accf) - reduce8(corr);
}

/* vecdot.zig:572-597 dotIQ4XS: per 32-weight sub-block the signed codebook dot (dps lanes) times
 * its scale, then one fma per super-block. */
static float dot_iq4_xs(const uint8_t *row, size_t nsb, const hko_block_q8k *a) {
    float accf[8] = {0};
    int32_t w[32], t0[8];
    for (size_t i = 0; i < nsb; i++) {
        const uint8_t *b = row + i * 136;
        int32_t acci[8] = {0};
        for (int ib = 0; ib < 8; ib++) {
            const uint8_t *qs = b + 8 + 16 * ib;
            for (int j = 0; j < 16; j++) {
                w[j] = kvalues_iq4nl[qs[j] & 0x0F];
                w[j + 16] = kvalues_iq4nl[qs[j] >> 4];
            }
            dp32(t0, w, a[i].qs + 32 * ib);
            int32_t ls = iq4xs_ls(b, ib);
            for (int L = 0; L < 8; L++) acci[L] += t0[L] * ls;
        }
        float s = h16(b) * a[i].d;
        for (int L = 0; L < 8; L++) accf[L] = fmaf((float)acci[L], s, accf[L]);
    }
    return reduce8(accf);
}

/* vecdot.zig:533-570 dotQ6K */
static float dot_q6_k(const uint8_t *row, size_t nsb, const hko_block_q8k *a) {
    float accf[8] = {0};
    int32_t qv[4][32], t0[8];
    for (size_t i = 0; i < nsb; i++) {
        const uint8_t *b = row + i * 210;
        const uint8_t *ql = b, *qh = b + 128;
        const int8_t *sc = (const int8_t *)(b + 192);
        int32_t acci[8] = {0};
        for (int half = 0; half < 2; half++) {
            const uint8_t *l0 = ql + half * 64, *l1 = ql + half * 64 + 32, *h = qh + half * 32;
            for (int j = 0; j < 32; j++) {
                qv[0][j] = (l0[j] & 0x0F) | ((h[j] & 3) << 4);
                qv[1][j] = (l1[j] & 0x0F) | (((h[j] >> 2) & 3) << 4);
                qv[2][j] = (l0[j] >> 4) | (((h[j] >> 4) & 3) << 4);
                qv[3][j] = (l1[j] >> 4) | (((h[j] >> 6) & 3) << 4);
            }
            for (int g = 0; g < 4; g++) {
                dp32(t0, qv[g], a[i].qs + half * 128 + g * 32);
                for (int L = 0; L < 8; L++) acci[L] += t0[L] * sc[8 * half + 2 * g + (L >= 4)];
            }
        }
        float s = h16(b + 208) * a[i].d;
        for (int L = 0; L < 8; L++) {
            int32_t bias = (a[i].bsums[2 * L] * sc[2 * L] + a[i].bsums[2 * L + 1] * sc[2 * L + 1]) * 32;
            accf[L] = fmaf((float)(acci[L] - bias), s, accf[L]);
        }
    }
    return reduce8(accf);
}

float hko_dot_row(int t, const uint8_t *row, size_t k, const hko_block_a8 *a8, const hko_block_q8k *q8k) {
    switch (t) {
    case HKO_Q8_0: case HKO_IQ4_NL: return dot_legacy(t, row, k / 32, a8);
    case HKO_Q4_0: case HKO_Q4_1: case HKO_Q5_0: case HKO_Q5_1: return dot_low_bit(t, row, k / 32, a8);
    case HKO_Q4_K: case HKO_Q5_K: return dot_q4_k(t, row, k / QK_K, q8k);
    case HKO_IQ4_XS: return dot_iq4_xs(row, k / QK_K, q8k);
    case HKO_Q6_K: return dot_q6_k(row, k / QK_K, q8k);
    default: return NAN;
    }
}

/* ---------------------------------------------------------------------------------------------
 * Register-tiled batch GEMM (gemm.zig). One output row is one SIMD lane there, so every
 * integer sum below is a whole-block (legacy) or whole-super-block (K) sum, and the float
 * update per block is two fused multiply-adds (gemm.zig:170-173, 225-231).
 * ------------------------------------------------------------------------------------------- */

/* unpack.zig:81-160 for Q4_K and Q6_K: vals unsigned, sc and mn per 16 weights. */
typedef struct {
    int16_t vals[256]; /* unsigned quants, or IQ4_XS's signed codebook values */
    int32_t sc[16], mn[16];
    float d, e;
} kblock;

static void unpack_k(int t, const uint8_t *b, kblock *o) {
    if (t == HKO_IQ4_XS) { /* unpack.zig:160-179: signed codebook values, no mins */
        o->d = o->e = h16(b);
        for (int ib = 0; ib < 8; ib++) {
            o->sc[2 * ib] = o->sc[2 * ib + 1] = iq4xs_ls(b, ib);
            o->mn[2 * ib] = o->mn[2 * ib + 1] = 0;
            for (int j = 0; j < 16; j++) {
                o->vals[32 * ib + j] = kvalues_iq4nl[b[8 + 16 * ib + j] & 0x0F];
                o->vals[32 * ib + j + 16] = kvalues_iq4nl[b[8 + 16 * ib + j] >> 4];
            }
        }
    } else if (t == HKO_Q4_K || t == HKO_Q5_K) { /* unpack.zig:118-139 */
        const int five = t == HKO_Q5_K, qoff = five ? 48 : 16;
        o->d = h16(b);
        o->e = h16(b + 2);
        for (int j = 0; j < 8; j++) {
            uint8_t sc, mn;
            hko_scale_min_k4(j, b + 4, &sc, &mn);
            o->sc[2 * j] = o->sc[2 * j + 1] = sc;
            o->mn[2 * j] = o->mn[2 * j + 1] = mn;
        }
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) {
                o->vals[64 * c + l] = (b[qoff + 32 * c + l] & 0x0F) + (five && ((b[16 + l] >> (2 * c)) & 1) ? 16 : 0);
                o->vals[64 * c + 32 + l] = (b[qoff + 32 * c + l] >> 4) + (five && ((b[16 + l] >> (2 * c + 1)) & 1) ? 16 : 0);
            }
    } else {
        const uint8_t *ql = b, *qh = b + 128;
        const int8_t *scales = (const int8_t *)(b + 192);
        o->d = o->e = h16(b + 208);
        for (int g = 0; g < 16; g++) {
            o->sc[g] = scales[g];
            o->mn[g] = 32 * scales[g];
        }
        for (int n = 0; n < 2; n++)
            for (int l = 0; l < 32; l++) {
                uint8_t h8 = qh[32 * n + l], a0 = ql[64 * n + l], a1 = ql[64 * n + l + 32];
                o->vals[128 * n + l] = (a0 & 0x0F) | ((h8 & 3) << 4);
                o->vals[128 * n + l + 32] = (a1 & 0x0F) | (((h8 >> 2) & 3) << 4);
                o->vals[128 * n + l + 64] = (a0 >> 4) | (((h8 >> 4) & 3) << 4);
                o->vals[128 * n + l + 96] = (a1 >> 4) | (((h8 >> 6) & 3) << 4);
            }
    }
}

/* gemm.zig:180-236 kernelK for one row against one token. */
static float tile_k(int t, const uint8_t *row, size_t nsb, const hko_block_q8k *a) {
    float accf = 0.0f;
    kblock kb;
    for (size_t s = 0; s < nsb; s++) {
        unpack_k(t, row + s * (size_t)hko_block_bytes(t), &kb);
        int32_t acc_sb = 0, acc_mn = 0;
        for (int g = 0; g < 16; g++) {
            int32_t d4 = 0;
            for (int k = 0; k < 16; k++) d4 += (int32_t)kb.vals[16 * g + k] * a[s].qs[16 * g + k];
            acc_sb += d4 * kb.sc[g];
        }
        for (int g = 0; g < 16; g++) acc_mn += kb.mn[g] * a[s].bsums[g];
        float dy = a[s].d;
        accf = fmaf((float)acc_sb, kb.d * dy, accf);
        accf = fmaf((float)acc_mn, -(kb.e * dy), accf);
    }
    return accf;
}

/* gemm.zig:131-176 kernelLegacy for one row and token: integer block sum of the unsigned quants,
 * minus zp * s, times d * d_a; plus m * (d_a * s) for the formats with an offset. */
static float tile_low_bit(int t, const uint8_t *row, size_t nb, const hko_block_a8 *a) {
    float accf = 0.0f;
    int32_t u[32];
    const int zp = low_bit_zp(t), has_m = low_bit_has_m(t);
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = row + i * (size_t)hko_block_bytes(t);
        low_bit_quants(t, b, u);
        int32_t acci = 0;
        for (int j = 0; j < 32; j++) acci += u[j] * a[i].qs[j];
        acci -= zp * a[i].s;
        accf = fmaf((float)acci, h16(b) * a[i].d, accf);
        if (has_m) accf = fmaf(h16(b + 2), a[i].d * (float)a[i].s, accf);
    }
    return accf;
}

/* gemm.zig:131-176 kernelLegacy (signed, no zero point, no offset) for one row and token. */
static float tile_legacy(int t, const uint8_t *row, size_t nb, const hko_block_a8 *a) {
    if (t != HKO_Q8_0 && t != HKO_IQ4_NL) return tile_low_bit(t, row, nb, a);
    float accf = 0.0f;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = row + i * (size_t)hko_block_bytes(t);
        int32_t acci = 0;
        for (int j = 0; j < 32; j++) {
            int32_t w = t == HKO_Q8_0 ? (int8_t)b[2 + j]
                                      : kvalues_iq4nl[j < 16 ? (b[2 + j] & 0x0F) : (b[2 + j - 16] >> 4)];
            acci += w * a[i].qs[j];
        }
        accf = fmaf((float)acci, h16(b) * a[i].d, accf);
    }
    return accf;
}

/* ---------------------------------------------------------------------------------------------
 * Matmul driver (abi_ops.zig:65-103, matmul.zig:96-153, kernels_impl.zig:14-33, gemm.zig:504-520)
 * ------------------------------------------------------------------------------------------- */

#include <stdlib.h>

int hko_matmul_path(int t, const uint8_t *w, size_t m, size_t k, const float *x, size_t n,
                    const float *bias, float *y, int threads, int tiled) {
    if (hko_fb_block_elems(t)) return hko_fb_matmul(t, w, m, k, x, n, bias, y, threads);
    int elems = hko_block_elems(t), kind = hko_act_kind(t);
    if (!elems || kind < 0) return -1;
    if (k % (size_t)elems || k % 32) return -2;
    if (m == 0 || n == 0) return 0;
    size_t row_bytes = k / (size_t)elems * (size_t)hko_block_bytes(t);
    hko_block_a8 *a8 = NULL;
    hko_block_q8k *qk = NULL;
    if (kind == 0) {
        a8 = (hko_block_a8 *)malloc(n * (k / 32) * sizeof(hko_block_a8));
        if (!a8) return -3;
        for (size_t i = 0; i < n; i++) hko_quantize_a8(x + i * k, k, a8 + i * (k / 32));
    } else {
        qk = (hko_block_q8k *)malloc(n * (k / QK_K) * sizeof(hko_block_q8k));
        if (!qk) return -3;
        for (size_t i = 0; i < n; i++) hko_quantize_q8k(x + i * k, k, qk + i * (k / QK_K));
    }
    long mm = (long)m;
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads > 0 ? threads : 1)
    for (long r = 0; r < mm; r++) {
        const uint8_t *row = w + (size_t)r * row_bytes;
        float b = bias ? bias[r] : 0.0f;
        for (size_t i = 0; i < n; i++) {
            float v;
            if (tiled)
                v = kind == 0 ? tile_legacy(t, row, k / 32, a8 + i * (k / 32))
                              : tile_k(t, row, k / QK_K, qk + i * (k / QK_K));
            else
                v = hko_dot_row(t, row, k, a8 ? a8 + i * (k / 32) : NULL, qk ? qk + i * (k / QK_K) : NULL);
            y[i * m + (size_t)r] = v + b;
        }
    }
    free(a8);
    free(qk);
    return 0;
}

int hko_matmul(int t, const uint8_t *w, size_t m, size_t k, const float *x, size_t n,
               const float *bias, float *y, int threads) {
    /* matmul.zig:18 min_tiled_tokens = 8 */
    return hko_matmul_path(t, w, m, k, x, n, bias, y, threads, n >= 8);
}
