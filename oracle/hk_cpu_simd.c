/* hk's CPU decode kernel for Q4_K with its SIMD instruction paths, for the benchmark's CPU
 * baseline. TEST / BASELINE INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg and tests/ call it;
 * the HIP product never does.
 *
 * What it restates:
 *  - the integer dot primitive dpu of src/quant/isa.zig:60-88: acc[i] += sum of the four products
 *    a[4i+k]*b[4i+k] (a unsigned <= 127, b signed), as one vpdpbusd on VNNI machines or
 *    vpmaddubsw + vpmaddwd on AVX2 (exact under those bounds), else a portable loop;
 *  - k4Block / dotQ4K of src/quant/vecdot.zig:461-522 on eight i32 / f32 lanes (per 64-weight
 *    pair of sub-blocks: acci += dpu(lo)*sc[2p] + dpu(hi)*sc[2p+1]; per super-block accf +=
 *    f32(acci)*(d*a.d), corr += f32(dotsum(bsums, dup16(mins)))*(dmin*a.d); the result is
 *    reduce(accf) - reduce(corr));
 *  - the decode partition of src/engine/matmul.zig:142-147: rows handed out in chunks of
 *    16 KiB of weights;
 *  - the run-time choice of the best instruction set the processor has
 *    (src/kernels.zig:55-85: avx512-vnni, avx2-vnni, avx2, generic), overridable by name.
 * The lane order and the final eight-lane sums are the same as in hk_oracle.c's dot_q4_k, so
 * every level gives the oracle's result bit for bit.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "hk_oracle.h"

#define QK_K 256
#define Q4K_BYTES 144

static inline float h16f(const uint8_t *p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return hko_f16_to_f32(h);
}

static inline float reduce8f(const float v[8]) {
    float s = v[0];
    for (int L = 1; L < 8; L++) s += v[L];
    return s;
}

/* ---- generic level (isa.zig dpEmulated) ---- */
static float dot_q4k_generic(const uint8_t *row, size_t nsb, const hko_block_q8k *a) {
    float accf[8] = {0}, corr[8] = {0};
    for (size_t i = 0; i < nsb; i++) {
        const uint8_t *b = row + i * Q4K_BYTES;
        uint8_t sc[8], mn[8];
        hko_scales_mins_k4_words(b + 4, sc, mn);
        int32_t acci[8] = {0};
        for (int p = 0; p < 4; p++) {
            const uint8_t *q = b + 16 + 32 * p;
            const int8_t *alo = a[i].qs + 64 * p, *ahi = alo + 32;
            for (int L = 0; L < 8; L++) {
                int32_t t0 = 0, t1 = 0;
                for (int k = 0; k < 4; k++) {
                    t0 += (q[4 * L + k] & 0x0F) * alo[4 * L + k];
                    t1 += (q[4 * L + k] >> 4) * ahi[4 * L + k];
                }
                acci[L] += t0 * sc[2 * p] + t1 * sc[2 * p + 1];
            }
        }
        const float sd = h16f(b) * a[i].d, sm = h16f(b + 2) * a[i].d;
        for (int L = 0; L < 8; L++) {
            const int32_t cs = a[i].bsums[2 * L] * mn[L] + a[i].bsums[2 * L + 1] * mn[L];
            accf[L] = fmaf((float)acci[L], sd, accf[L]);
            corr[L] = fmaf((float)cs, sm, corr[L]);
        }
    }
    return reduce8f(accf) - reduce8f(corr);
}

/* ---- the x86 levels: one body, the dot primitive chosen by the target ---- */
#define DOT_Q4K_BODY(DPU)                                                                            \
    __m256 accf = _mm256_setzero_ps(), corr = _mm256_setzero_ps();                                   \
    const __m256i m4 = _mm256_set1_epi8(0x0F);                                                       \
    for (size_t i = 0; i < nsb; i++) {                                                               \
        const uint8_t *b = row + i * Q4K_BYTES;                                                      \
        uint8_t sc[8], mn[8];                                                                        \
        hko_scales_mins_k4_words(b + 4, sc, mn);                                                     \
        __m256i acci = _mm256_setzero_si256();                                                       \
        for (int p = 0; p < 4; p++) {                                                                \
            const __m256i q = _mm256_loadu_si256((const __m256i *)(b + 16 + 32 * p));                \
            const __m256i lo = _mm256_and_si256(q, m4);                                              \
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);                       \
            const __m256i alo = _mm256_loadu_si256((const __m256i *)(a[i].qs + 64 * p));             \
            const __m256i ahi = _mm256_loadu_si256((const __m256i *)(a[i].qs + 64 * p + 32));        \
            const __m256i t0 = DPU(lo, alo), t1 = DPU(hi, ahi);                                      \
            acci = _mm256_add_epi32(acci, _mm256_add_epi32(_mm256_mullo_epi32(t0, _mm256_set1_epi32(sc[2 * p])), \
                                                            _mm256_mullo_epi32(t1, _mm256_set1_epi32(sc[2 * p + 1])))); \
        }                                                                                            \
        const __m256i bs = _mm256_loadu_si256((const __m256i *)a[i].bsums);                          \
        const __m256i mins = _mm256_setr_epi16(mn[0], mn[0], mn[1], mn[1], mn[2], mn[2], mn[3], mn[3], \
                                               mn[4], mn[4], mn[5], mn[5], mn[6], mn[6], mn[7], mn[7]); \
        const __m256i cs = _mm256_madd_epi16(bs, mins);                                              \
        const float sd = h16f(b) * a[i].d, sm = h16f(b + 2) * a[i].d;                                \
        accf = _mm256_fmadd_ps(_mm256_cvtepi32_ps(acci), _mm256_set1_ps(sd), accf);                  \
        corr = _mm256_fmadd_ps(_mm256_cvtepi32_ps(cs), _mm256_set1_ps(sm), corr);                    \
    }                                                                                                \
    float fa[8], fc[8];                                                                              \
    _mm256_storeu_ps(fa, accf);                                                                      \
    _mm256_storeu_ps(fc, corr);                                                                      \
    return reduce8f(fa) - reduce8f(fc);

__attribute__((target("avx2,fma"))) static inline __m256i dpu_avx2(__m256i u, __m256i s) {
    const __m256i m = _mm256_maddubs_epi16(u, s); /* exact: u <= 15 here, far below 127 */
    return _mm256_madd_epi16(m, _mm256_set1_epi16(1));
}
__attribute__((target("avx2,fma"))) static float dot_q4k_avx2(const uint8_t *row, size_t nsb, const hko_block_q8k *a) {
    DOT_Q4K_BODY(dpu_avx2)
}

__attribute__((target("avx2,fma,avxvnni"))) static inline __m256i dpu_avxvnni(__m256i u, __m256i s) {
    return _mm256_dpbusd_avx_epi32(_mm256_setzero_si256(), u, s);
}
__attribute__((target("avx2,fma,avxvnni"))) static float dot_q4k_avxvnni(const uint8_t *row, size_t nsb,
                                                                         const hko_block_q8k *a) {
    DOT_Q4K_BODY(dpu_avxvnni)
}

__attribute__((target("avx2,fma,avx512f,avx512vl,avx512vnni"))) static inline __m256i dpu_avx512vnni(__m256i u, __m256i s) {
    return _mm256_dpbusd_epi32(_mm256_setzero_si256(), u, s);
}
__attribute__((target("avx2,fma,avx512f,avx512vl,avx512vnni"))) static float dot_q4k_avx512vnni(const uint8_t *row, size_t nsb,
                                                                                              const hko_block_q8k *a) {
    DOT_Q4K_BODY(dpu_avx512vnni)
}

typedef float (*dot_fn)(const uint8_t *, size_t, const hko_block_q8k *);

static const struct {
    const char *name;
    dot_fn fn;
} LEVELS[] = {
    {"avx512-vnni", dot_q4k_avx512vnni},
    {"avx2-vnni", dot_q4k_avxvnni},
    {"avx2", dot_q4k_avx2},
    {"generic", dot_q4k_generic},
};

static int supported(int level) {
    __builtin_cpu_init();
    switch (level) {
    case 0: return __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl");
    case 1: return __builtin_cpu_supports("avxvnni") && __builtin_cpu_supports("avx2");
    case 2: return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    default: return 1;
    }
}

/* Best level this processor runs, or the one named (if it runs here); -1 if the name is unknown
 * or unsupported. */
int hkc_pick_level(const char *name) {
    for (int l = 0; l < 4; l++) {
        if (name && strcmp(name, LEVELS[l].name) != 0) continue;
        if (supported(l)) return l;
        if (name) return -1;
    }
    return -1;
}

const char *hkc_level_name(int level) { return level >= 0 && level < 4 ? LEVELS[level].name : ""; }

/* y[r] = dot(W[r], x) for a Q4_K matrix m x k and one token: x quantized with quantizeQ8K, rows
 * in 16 KiB chunks over `threads` OpenMP threads. Returns 0, or -1 for a bad level / shape. */
int hkc_matvec_q4k(int level, const uint8_t *w, size_t m, size_t k, const float *x, float *y, int threads) {
    if (level < 0 || level >= 4 || !supported(level) || k % QK_K) return -1;
    const size_t nsb = k / QK_K, row_bytes = nsb * Q4K_BYTES;
    hko_block_q8k *a = (hko_block_q8k *)malloc(nsb * sizeof(hko_block_q8k));
    if (!a) return -1;
    hko_quantize_q8k(x, k, a);
    const dot_fn fn = LEVELS[level].fn;
    long grain = (long)(16384 / row_bytes);
    if (grain < 1) grain = 1;
    const long mm = (long)m;
#pragma omp parallel for schedule(dynamic, grain) num_threads(threads > 0 ? threads : 1)
    for (long r = 0; r < mm; r++) y[r] = fn(w + (size_t)r * row_bytes, nsb, a);
    free(a);
    return 0;
}
