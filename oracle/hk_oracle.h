/* CPU oracle for hk's quantized-linear hot path. TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of hk's CPU kernels (Zig sources under src/quant/ and
 * src/engine/matmul.zig of the reference). It is the checker that the HIP
 * library is compared against, and the "port" CPU baseline timed by bench.py.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it; nothing in hk_amd/ links or calls it.
 *
 * Every routine works on the file layout of the blocks (GGML byte layouts,
 * reference src/quant/blocks.zig:17-34), little endian.
 */
#ifndef HK_ORACLE_H
#define HK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hk StorageType codes (reference src/format.zig:26-84). */
#define HKO_Q4_0 0x15
#define HKO_Q8_0 0x16
#define HKO_Q4_1 0x17
#define HKO_Q5_0 0x18
#define HKO_Q5_1 0x19
#define HKO_Q4_K 0x42
#define HKO_Q5_K 0x43
#define HKO_Q6_K 0x44
#define HKO_IQ4_NL 0x55
#define HKO_IQ4_XS 0x56
/* Formats hk decodes to floats before its dots (src/format.zig:71-93). */
#define HKO_Q2_K 0x40
#define HKO_Q3_K 0x41
#define HKO_IQ1_S 0x50
#define HKO_IQ1_M 0x51
#define HKO_IQ2_XXS 0x52
#define HKO_IQ2_XS 0x53
#define HKO_IQ3_XXS 0x54
#define HKO_IQ2_S 0x57
#define HKO_IQ3_S 0x58
#define HKO_TQ1_0 0x60
#define HKO_TQ2_0 0x61
#define HKO_MXFP4 0x62
#define HKO_NVFP4 0x63

/* Activation blocks, byte-identical to the reference structs. */
typedef struct {
    float d;
    int32_t s;
    int8_t qs[32];
} hko_block_a8; /* vecdot.zig:22-26, 40 bytes */

typedef struct {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} hko_block_q8k; /* blocks.zig:25, 292 bytes */

/* Block geometry: weights per block and bytes per block; 0 when unsupported. */
int hko_block_elems(int t);
int hko_block_bytes(int t);

/* f16 bits to f32, exact. */
float hko_f16_to_f32(uint16_t h);

/* dequant.zig:550 dequantizeRow for the four formats; returns 0 or -1 (BadLength / type). */
int hko_dequantize_row(int t, const uint8_t *src, size_t src_len, float *dst, size_t n);

/* vecdot.zig:134-180. */
void hko_quantize_a8(const float *x, size_t n, hko_block_a8 *out);
void hko_quantize_q8k(const float *x, size_t n, hko_block_q8k *out);

/* vecdot.zig:185 actKind: 0 = A8, 1 = Q8K, -1 = unsupported. */
int hko_act_kind(int t);

/* vecdot.zig:725-771 dotRow: one row against one prepared activation. */
float hko_dot_row(int t, const uint8_t *row, size_t k, const hko_block_a8 *a8, const hko_block_q8k *q8k);

/* scalesMinsK4 (vecdot.zig:461-474), the word trick, exposed so tests can pin it
 * against scaleMinK4 (dequant.zig:166-175). */
void hko_scales_mins_k4_words(const uint8_t packed12[12], uint8_t sc[8], uint8_t mn[8]);
void hko_scale_min_k4(int j, const uint8_t packed12[12], uint8_t *sc, uint8_t *mn);

/* y[t*m + r] = dot(W[r], x[t]) + bias[r] for n tokens, exactly as abi_ops.gemm
 * (engine/abi_ops.zig:65-103) drives matmul.run: n >= 8 uses the register-tiled
 * batch kernel arithmetic (gemm.zig), fewer tokens the row kernels (vecdot.zig).
 * `threads` > 1 splits rows over OpenMP threads (the CPU baseline). Returns 0 or
 * a negative error (-1 type, -2 shape). */
int hko_matmul(int t, const uint8_t *w, size_t m, size_t k, const float *x, size_t n,
               const float *bias, float *y, int threads);

/* Force one of the two CPU paths regardless of n: 0 = rows (vecdot), 1 = tiles (gemm). */
int hko_matmul_path(int t, const uint8_t *w, size_t m, size_t k, const float *x, size_t n,
                    const float *bias, float *y, int threads, int tiled);

/* hk_oracle_fallback.c: geometry, activation kind (0 A8, 1 Q8K, 2 f32), one block decoded to
 * floats (bit-exact), and the products (float64 restatement of hk's dots). */
int hko_fb_block_elems(int t);
int hko_fb_block_bytes(int t);
int hko_fb_act_kind(int t);
int hko_fb_decode_block(int t, const uint8_t *b, float *out);
int hko_fb_matmul(int t, const uint8_t *w, size_t m, size_t k, const float *x, size_t n, const float *bias, float *y,
                  int threads);

#ifdef __cplusplus
}
#endif
#endif
