/* CPU oracle, part 2: the formats hk decodes to floats before its dot products (TEST
 * INFRASTRUCTURE ONLY, like hk_oracle.c): Q2_K, Q3_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S,
 * IQ1_S, IQ1_M, TQ1_0, TQ2_0, MXFP4, NVFP4.
 *
 * Decoders restate src/quant/dequant.zig (q2_k 80-112, q3kScales 114-128, q3_k 130-165,
 * iq2_xxs 278-294, iq2_xs 296-312, iq2_s 314-330, iq3_xxs 332-351, iq3_s 353-375, iq1_s 377-392,
 * iq1_m 394-428, ternary / tq1_0 460-488, tq2_0 490-504, e8m0Half / mxfp4 506-519, ue4m3Half /
 * nvfp4 521-548) operation by operation (built with -ffp-contract=off), so they are bit-exact.
 * Products: hk computes them as exact integer dots of canonical weights against the Q8K / A8
 * activations (vecdot.zig dotCanonK 686-705, dotCanonLegacy 707-720) or, for NVFP4, as f32 dots
 * of the decoded block against the f32 input (dotGeneric 620-631). The oracle evaluates the
 * same sums in float64 from the decoded weights and the dequantized activations (d * q), which is
 * algebraically the integer dot: equal up to the final f32 rounding.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "hk_oracle.h"
#include "_gen/iq_tables.h"

static float f16f(const uint8_t *p) { return hko_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }
static uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ksigns_iq2xs: the 7 sign bits plus an 8th that makes the count even (a parity table). */
static uint8_t ksign(uint32_t i) { return (uint8_t)(i | ((__builtin_popcount(i) & 1) << 7)); }
static float sign_of(uint8_t s, int j) { return (s >> j) & 1 ? -1.0f : 1.0f; } /* kmask_iq2xs = 1 << j */

static const int8_t kvalues_fp4[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12}; /* tables.zig:16 */
static const float iq1s_delta = 0.125f;                                                       /* tables.zig:18 */

int hko_fb_block_elems(int t) {
    switch (t) {
    case HKO_MXFP4: return 32;
    case HKO_NVFP4: return 64;
    case HKO_Q2_K: case HKO_Q3_K: case HKO_IQ2_XXS: case HKO_IQ2_XS: case HKO_IQ2_S: case HKO_IQ3_XXS:
    case HKO_IQ3_S: case HKO_IQ1_S: case HKO_IQ1_M: case HKO_TQ1_0: case HKO_TQ2_0: return 256;
    default: return 0;
    }
}

int hko_fb_block_bytes(int t) { /* blocks.zig:19-40 */
    switch (t) {
    case HKO_Q2_K: return 84;
    case HKO_Q3_K: return 110;
    case HKO_IQ2_XXS: return 66;
    case HKO_IQ2_XS: return 74;
    case HKO_IQ2_S: return 82;
    case HKO_IQ3_XXS: return 98;
    case HKO_IQ3_S: return 110;
    case HKO_IQ1_S: return 50;
    case HKO_IQ1_M: return 56;
    case HKO_TQ1_0: return 54;
    case HKO_TQ2_0: return 66;
    case HKO_MXFP4: return 17;
    case HKO_NVFP4: return 36;
    default: return 0;
    }
}

int hko_fb_act_kind(int t) { /* vecdot.zig:185-191 */
    if (t == HKO_MXFP4) return 0;
    if (t == HKO_NVFP4) return 2;
    return hko_fb_block_elems(t) ? 1 : -1;
}

static void deq_q2_k(const uint8_t *b, float *out) { /* {scales[16], qs[64], d, dmin} */
    const float d = f16f(b + 80), min = f16f(b + 82);
    int is = 0, o = 0, q = 0;
    for (int n = 0; n < 256; n += 128) {
        int shift = 0;
        for (int it = 0; it < 4; it++) {
            for (int half = 0; half < 2; half++) {
                const uint8_t sc = b[is++];
                const float dl = d * (float)(sc & 0x0F), ml = min * (float)(sc >> 4);
                for (int l = 0; l < 16; l++) out[o++] = dl * (float)((b[16 + q + l + 16 * half] >> shift) & 3) - ml;
            }
            shift += 2;
        }
        q += 32;
    }
}

static void q3k_scales(const uint8_t *p, int8_t scales[16]) {
    const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0f0f0f0fu;
    uint32_t aux[4] = {rd32(p), rd32(p + 4), rd32(p + 8), 0};
    const uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
    aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
    aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
    aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
    for (int i = 0; i < 4; i++)
        for (int k = 0; k < 4; k++) scales[4 * i + k] = (int8_t)(aux[i] >> (8 * k));
}

static void deq_q3_k(const uint8_t *b, float *out) { /* {hmask[32], qs[64], scales[12], d} */
    const float d_all = f16f(b + 108);
    int8_t scales[16];
    q3k_scales(b + 96, scales);
    int is = 0, o = 0, q = 0;
    uint8_t m = 1;
    for (int n = 0; n < 256; n += 128) {
        int shift = 0;
        for (int it = 0; it < 4; it++) {
            for (int half = 0; half < 2; half++) {
                const float dl = d_all * (float)((int)scales[is++] - 32);
                for (int l = 0; l < 16; l++) {
                    const int lo = (b[32 + q + l + 16 * half] >> shift) & 3;
                    const int hi = (b[l + 16 * half] & m) ? 0 : 4;
                    out[o++] = dl * (float)(lo - hi);
                }
            }
            shift += 2;
            m <<= 1;
        }
        q += 32;
    }
}

static void deq_iq2_xxs(const uint8_t *b, float *out) { /* {d, qs[64]} */
    const float d = f16f(b);
    const uint8_t *qs = b + 2;
    int o = 0;
    for (int ib = 0; ib < 8; ib++) {
        const uint32_t aux1 = rd32(qs + 8 * ib + 4);
        const float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            const uint8_t *grid = iq2xxs_grid + 8 * qs[8 * ib + l];
            const uint8_t signs = ksign((aux1 >> (7 * l)) & 127);
            for (int j = 0; j < 8; j++) out[o + j] = db * (float)grid[j] * sign_of(signs, j);
            o += 8;
        }
    }
}

static void deq_iq2_xs(const uint8_t *b, float *out) { /* {d, qs[64] (u16 x 32), scales[8]} */
    const float d = f16f(b);
    int o = 0;
    for (int ib = 0; ib < 8; ib++) {
        const uint8_t sc = b[66 + ib];
        const float db0 = d * (0.5f + (float)(sc & 0x0F)) * 0.25f, db1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            const uint16_t q = rd16(b + 2 + 2 * (4 * ib + l));
            const uint8_t *grid = iq2xs_grid + 8 * (q & 511);
            const uint8_t signs = ksign(q >> 9);
            const float db = l < 2 ? db0 : db1;
            for (int j = 0; j < 8; j++) out[o + j] = db * (float)grid[j] * sign_of(signs, j);
            o += 8;
        }
    }
}

static void deq_iq2_s(const uint8_t *b, float *out) { /* {d, qs[32], signs[32], qh[8], scales[8]} */
    const float d = f16f(b);
    int o = 0;
    for (int ib = 0; ib < 8; ib++) {
        const uint8_t sc = b[74 + ib];
        const float db0 = d * (0.5f + (float)(sc & 0x0F)) * 0.25f, db1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            const uint32_t hi = ((uint32_t)b[66 + ib] << (8 - 2 * l)) & 0x300;
            const uint8_t *grid = iq2s_grid + 8 * (b[2 + 4 * ib + l] | hi);
            const uint8_t signs = b[34 + 4 * ib + l];
            const float db = l < 2 ? db0 : db1;
            for (int j = 0; j < 8; j++) out[o + j] = db * (float)grid[j] * sign_of(signs, j);
            o += 8;
        }
    }
}

static void deq_iq3_xxs(const uint8_t *b, float *out) { /* {d, qs[96]} */
    const float d = f16f(b);
    const uint8_t *qs = b + 2;
    int o = 0;
    for (int ib = 0; ib < 8; ib++) {
        const uint32_t aux = rd32(qs + 64 + 4 * ib);
        const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
        for (int l = 0; l < 4; l++) {
            const uint8_t signs = ksign((aux >> (7 * l)) & 127);
            const uint8_t *g1 = iq3xxs_grid + 4 * qs[8 * ib + 2 * l], *g2 = iq3xxs_grid + 4 * qs[8 * ib + 2 * l + 1];
            for (int j = 0; j < 4; j++) {
                out[o + j] = db * (float)g1[j] * sign_of(signs, j);
                out[o + j + 4] = db * (float)g2[j] * sign_of(signs, j + 4);
            }
            o += 8;
        }
    }
}

static void deq_iq3_s(const uint8_t *b, float *out) { /* {d, qs[64], qh[8], signs[32], scales[4]} */
    const float d = f16f(b);
    const uint8_t *qs = b + 2, *qh = b + 66, *signs = b + 74, *scales = b + 106;
    int o = 0;
    for (int g = 0; g < 32; g++) {
        const uint32_t nib = (scales[g / 8] >> (4 * ((g / 4) & 1))) & 0x0F;
        const float db = d * (float)(1 + 2 * nib);
        const int e0 = 2 * g, e1 = 2 * g + 1;
        const uint32_t i0 = qs[e0] | (((uint32_t)(qh[e0 / 8] >> (e0 % 8)) & 1) << 8);
        const uint32_t i1 = qs[e1] | (((uint32_t)(qh[e1 / 8] >> (e1 % 8)) & 1) << 8);
        const uint8_t *g1 = iq3s_grid + 4 * i0, *g2 = iq3s_grid + 4 * i1;
        for (int j = 0; j < 4; j++) {
            out[o + j] = db * (float)g1[j] * sign_of(signs[g], j);
            out[o + j + 4] = db * (float)g2[j] * sign_of(signs[g], j + 4);
        }
        o += 8;
    }
}

static void deq_iq1_s(const uint8_t *b, float *out) { /* {d, qs[32], qh[16]} */
    const float d = f16f(b);
    int o = 0;
    for (int ib = 0; ib < 8; ib++) {
        const uint16_t qh = rd16(b + 34 + 2 * ib);
        const float dl = d * (float)(2 * ((qh >> 12) & 7) + 1);
        const float delta = (qh & 0x8000) ? -iq1s_delta : iq1s_delta;
        for (int l = 0; l < 4; l++) {
            const uint32_t idx = b[2 + 4 * ib + l] | ((uint32_t)((qh >> (3 * l)) & 7) << 8);
            const int8_t *grid = (const int8_t *)iq1s_grid + 8 * idx;
            for (int j = 0; j < 8; j++) out[o + j] = dl * ((float)grid[j] + delta);
            o += 8;
        }
    }
}

static void deq_iq1_m(const uint8_t *b, float *out) { /* {qs[32], qh[16], scales[8]} */
    uint16_t sc[4];
    for (int i = 0; i < 4; i++) sc[i] = rd16(b + 48 + 2 * i);
    const uint16_t bits = (uint16_t)((sc[0] >> 12) | ((sc[1] >> 8) & 0x00F0) | ((sc[2] >> 4) & 0x0F00) | (sc[3] & 0xF000));
    const float d = hko_f16_to_f32(bits);
    int o = 0;
    for (int ib = 0; ib < 8; ib++) {
        const uint16_t w = sc[ib / 2];
        const int base = 6 * (ib % 2);
        const float dl1 = d * (float)(2 * ((w >> base) & 7) + 1), dl2 = d * (float)(2 * ((w >> (base + 3)) & 7) + 1);
        const uint8_t qh0 = b[32 + 2 * ib], qh1 = b[32 + 2 * ib + 1];
        const uint32_t idx[4] = {b[4 * ib] | (((uint32_t)qh0 << 8) & 0x700), b[4 * ib + 1] | (((uint32_t)qh0 << 4) & 0x700),
                                 b[4 * ib + 2] | (((uint32_t)qh1 << 8) & 0x700), b[4 * ib + 3] | (((uint32_t)qh1 << 4) & 0x700)};
        const float delta[4] = {(qh0 & 0x08) ? -iq1s_delta : iq1s_delta, (qh0 & 0x80) ? -iq1s_delta : iq1s_delta,
                                (qh1 & 0x08) ? -iq1s_delta : iq1s_delta, (qh1 & 0x80) ? -iq1s_delta : iq1s_delta};
        for (int l = 0; l < 4; l++) {
            const float dl = l < 2 ? dl1 : dl2;
            const int8_t *grid = (const int8_t *)iq1s_grid + 8 * idx[l];
            for (int j = 0; j < 8; j++) out[o + j] = dl * ((float)grid[j] + delta[l]);
            o += 8;
        }
    }
}

static float ternary(uint8_t q, uint8_t mul) {
    const uint8_t v = (uint8_t)(q * mul);
    const uint32_t t = ((uint32_t)v * 3) >> 8;
    return (float)((int)t - 1);
}

static void deq_tq1_0(const uint8_t *b, float *out) { /* {qs[48], qh[4], d} */
    static const uint8_t pow3[5] = {1, 3, 9, 27, 81};
    const float d = f16f(b + 52);
    int o = 0;
    for (int n = 0; n < 5; n++)
        for (int m = 0; m < 32; m++) out[o++] = ternary(b[m], pow3[n]) * d;
    for (int n = 0; n < 5; n++)
        for (int m = 0; m < 16; m++) out[o++] = ternary(b[32 + m], pow3[n]) * d;
    for (int n = 0; n < 4; n++)
        for (int m = 0; m < 4; m++) out[o++] = ternary(b[48 + m], pow3[n]) * d;
}

static void deq_tq2_0(const uint8_t *b, float *out) { /* {qs[64], d} */
    const float d = f16f(b + 64);
    int o = 0;
    for (int j = 0; j < 64; j += 32)
        for (int l = 0; l < 4; l++)
            for (int k = 0; k < 32; k++) out[o++] = (float)(((b[j + k] >> (2 * l)) & 3) - 1) * d;
}

static float e8m0_half(uint8_t e) {
    const uint32_t bits = e < 2 ? (0x00200000u << e) : ((uint32_t)e - 1) << 23;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static void deq_mxfp4(const uint8_t *b, float *out) { /* {e, qs[16]} */
    const float d = e8m0_half(b[0]);
    for (int j = 0; j < 16; j++) {
        out[j] = (float)kvalues_fp4[b[1 + j] & 0x0F] * d;
        out[j + 16] = (float)kvalues_fp4[b[1 + j] >> 4] * d;
    }
}

static float ue4m3_half(uint8_t x) {
    if (x == 0 || x == 0x7F) return 0.0f;
    const int e = (x >> 3) & 0xF;
    const float man = (float)(x & 7);
    float raw;
    if (e == 0) {
        raw = man * 0x1p-9f;
    } else {
        const uint32_t bits = (uint32_t)(e - 7 + 127) << 23;
        float p;
        memcpy(&p, &bits, 4);
        raw = (1.0f + man / 8.0f) * p;
    }
    return raw * 0.5f;
}

static void deq_nvfp4(const uint8_t *b, float *out) { /* {d[4], qs[32]} */
    for (int s = 0; s < 4; s++) {
        const float d = ue4m3_half(b[s]);
        for (int j = 0; j < 8; j++) {
            const uint8_t byte = b[4 + 8 * s + j];
            out[16 * s + j] = (float)kvalues_fp4[byte & 0x0F] * d;
            out[16 * s + 8 + j] = (float)kvalues_fp4[byte >> 4] * d;
        }
    }
}

int hko_fb_decode_block(int t, const uint8_t *b, float *out) {
    switch (t) {
    case HKO_Q2_K: deq_q2_k(b, out); return 0;
    case HKO_Q3_K: deq_q3_k(b, out); return 0;
    case HKO_IQ2_XXS: deq_iq2_xxs(b, out); return 0;
    case HKO_IQ2_XS: deq_iq2_xs(b, out); return 0;
    case HKO_IQ2_S: deq_iq2_s(b, out); return 0;
    case HKO_IQ3_XXS: deq_iq3_xxs(b, out); return 0;
    case HKO_IQ3_S: deq_iq3_s(b, out); return 0;
    case HKO_IQ1_S: deq_iq1_s(b, out); return 0;
    case HKO_IQ1_M: deq_iq1_m(b, out); return 0;
    case HKO_TQ1_0: deq_tq1_0(b, out); return 0;
    case HKO_TQ2_0: deq_tq2_0(b, out); return 0;
    case HKO_MXFP4: deq_mxfp4(b, out); return 0;
    case HKO_NVFP4: deq_nvfp4(b, out); return 0;
    default: return -1;
    }
}

/* y[t*m + r] = sum_k w[r][k] * act[t][k] + bias[r] in float64, act the dequantized Q8K / A8
 * activations (quantizeQ8K / quantizeA8 of x) or x itself (NVFP4). */
int hko_fb_matmul(int t, const uint8_t *w, size_t m, size_t k, const float *x, size_t n, const float *bias, float *y,
                  int threads) {
    const int elems = hko_fb_block_elems(t), bytes = hko_fb_block_bytes(t), kind = hko_fb_act_kind(t);
    if (!elems) return -1;
    if (k % (size_t)elems || (kind == 1 && k % 256) || (kind == 0 && k % 32)) return -2;
    double *act = (double *)malloc(n * k * sizeof(double));
    if (!act) return -3;
    for (size_t i = 0; i < n; i++) {
        const float *xi = x + i * k;
        double *ai = act + i * k;
        if (kind == 2) {
            for (size_t e = 0; e < k; e++) ai[e] = xi[e];
        } else if (kind == 1) {
            hko_block_q8k *qb = (hko_block_q8k *)malloc((k / 256) * sizeof(hko_block_q8k));
            hko_quantize_q8k(xi, k, qb);
            for (size_t e = 0; e < k; e++) ai[e] = (double)qb[e / 256].d * (double)qb[e / 256].qs[e % 256];
            free(qb);
        } else {
            hko_block_a8 *ab = (hko_block_a8 *)malloc((k / 32) * sizeof(hko_block_a8));
            hko_quantize_a8(xi, k, ab);
            for (size_t e = 0; e < k; e++) ai[e] = (double)ab[e / 32].d * (double)ab[e / 32].qs[e % 32];
            free(ab);
        }
    }
    const size_t nb = k / (size_t)elems, row_bytes = nb * (size_t)bytes;
    const long mm = (long)m;
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads > 0 ? threads : 1)
    for (long r = 0; r < mm; r++) {
        float wbuf[256];
        double acc[64];
        const size_t nn = n < 64 ? n : 64;
        for (size_t c0 = 0; c0 < n; c0 += nn) {
            const size_t cn = n - c0 < nn ? n - c0 : nn;
            for (size_t i = 0; i < cn; i++) acc[i] = 0.0;
            for (size_t b = 0; b < nb; b++) {
                hko_fb_decode_block(t, w + (size_t)r * row_bytes + b * (size_t)bytes, wbuf);
                for (size_t i = 0; i < cn; i++) {
                    const double *ai = act + (c0 + i) * k + b * (size_t)elems;
                    double s = 0.0;
                    for (int e = 0; e < elems; e++) s += (double)wbuf[e] * ai[e];
                    acc[i] += s;
                }
            }
            for (size_t i = 0; i < cn; i++) y[(c0 + i) * m + (size_t)r] = (float)acc[i] + (bias ? bias[r] : 0.0f);
        }
    }
    free(act);
    return 0;
}
