/* hkhip.h — C ABI of the MI355X (gfx950) quantized-linear engine for hk.
 *
 * This is the drop-in boundary a HIP backend of hk binds: hk's Zig host side would
 * @cImport this header the way src/cuda.zig loads libcuda, and a `hip` arm is added to
 * backend.Device (reference src/backend/backend.zig:27,128-209). Every entry point takes
 * plain pointers, sizes and hk's own StorageType byte codes (src/format.zig:26-84).
 *
 * Shapes follow hk's engine: W is `rows` x `cols` (M x K) in one of the block formats,
 * activations x are token major [n][K] f32, outputs y are token major [n][M] f32
 * (src/engine/matmul.zig:5, src/kernels_impl.zig:27).
 *
 * Error convention: entry points return 0 on success or a negative HKHIP_E_* code and
 * set a thread-local message readable with hkhip_last_error(). The codes mirror the CUDA
 * engine's error set (src/cuda/engine.zig:31-40). The host-pointer products
 * (hkhip_gemv_*, hkhip_gemm_host) additionally fill y with NaN on failure, as hk's C ABI
 * does (src/c_api.zig:16-18).
 *
 * Threading: one engine = one device + one stream. Calls on one engine are serialised by
 * the caller (hk's Model does this); every entry point makes the engine's device current,
 * so an engine may be used from a thread other than the one that created it.
 */
#ifndef HKHIP_H
#define HKHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hk StorageType codes handled by the HIP kernels (src/format.zig:49-53,75-77,84-85). */
#define HKHIP_Q4_0 0x15
#define HKHIP_Q8_0 0x16
#define HKHIP_Q4_1 0x17
#define HKHIP_Q5_0 0x18
#define HKHIP_Q5_1 0x19
#define HKHIP_Q4_K 0x42
#define HKHIP_Q5_K 0x43
#define HKHIP_Q6_K 0x44
#define HKHIP_IQ4_NL 0x55
#define HKHIP_IQ4_XS 0x56
/* Formats whose products decode the weights to floats first, hk's "exact fallback" (vecdot.zig
 * dotCanonK / dotCanonLegacy / dotGeneric): upload, bit-exact decode and products (1..8 tokens per
 * decode pass; longer inputs in passes), no MFMA GEMM (src/format.zig:71-93). */
#define HKHIP_Q2_K 0x40
#define HKHIP_Q3_K 0x41
#define HKHIP_IQ1_S 0x50
#define HKHIP_IQ1_M 0x51
#define HKHIP_IQ2_XXS 0x52
#define HKHIP_IQ2_XS 0x53
#define HKHIP_IQ3_XXS 0x54
#define HKHIP_IQ2_S 0x57
#define HKHIP_IQ3_S 0x58
#define HKHIP_TQ1_0 0x60
#define HKHIP_TQ2_0 0x61
#define HKHIP_MXFP4 0x62
#define HKHIP_NVFP4 0x63 /* dotted against the f32 input (vecdot.zig:189): products need x, not xq */

/* Activation kinds (src/quant/vecdot.zig:183-191 ActKind). */
#define HKHIP_ACT_A8 0  /* per 32: d = amax/127, round half away, s = sum q */
#define HKHIP_ACT_Q8K 1 /* per 256: signed-max scale, clamp 127, 16 bsums   */
#define HKHIP_ACT_F32 2 /* no quantization (NVFP4): products read the f32 input itself */

/* Output modes of the products. */
#define HKHIP_STORE 0      /* y  = W x + bias */
#define HKHIP_ACCUMULATE 1 /* y += W x + bias (residual add fused into the product) */
/* Fused gate/up of a SwiGLU FFN, the Vulkan engine's mmvq mode 2 (shaders/mmvq.comp:24,162-186):
 * W holds the gate and up rows interleaved (row 2i = gate i, row 2i + 1 = up i), y is [n][rows/2]
 * and y[t][i] = silu(g) * u with g, u the two rows' products, silu(g) = g / (1 + exp(-g)). Rows
 * even, no bias. Every product takes it; in the GEMMs (no counterpart in the reference, whose
 * prefill writes both rows and applies swiglu separately) it halves the output written. */
#define HKHIP_SILU_MUL 2

/* Error codes (src/cuda/engine.zig:31-40). */
#define HKHIP_OK 0
#define HKHIP_E_UNSUPPORTED_TYPE -1
#define HKHIP_E_UNSUPPORTED_SHAPE -2
#define HKHIP_E_OUT_OF_DEVICE_MEMORY -3
#define HKHIP_E_DEVICE_FAILED -4
#define HKHIP_E_BAD_ARGUMENT -5
#define HKHIP_E_NO_DEVICE -6

typedef struct hkhip_engine hkhip_engine;

/* A weight matrix resident on the device. The device layout is private to the engine
 * (Q4_K is kept in file layout; Q8_0, Q6_K and IQ4_NL are split into an aligned quant plane
 * and a scale plane); `file_bytes` is the size of the same matrix in hk's file layout.
 * Mirrors DevMat{mem, t, rows, cols} (src/cuda/engine.zig:111-116). */
typedef struct hkhip_mat {
    void *mem;
    uint64_t file_bytes;
    uint64_t dev_bytes;
    uint32_t rows;
    uint32_t cols;
    uint8_t t;
    uint8_t owned;
    uint8_t pad[6];
} hkhip_mat;

/* ---- engine lifetime (probeCuda / Engine.init / deinit: src/backend/backend.zig:92-126) ---- */
int hkhip_device_count(void);
int hkhip_init(int device, hkhip_engine **out);
void hkhip_destroy(hkhip_engine *eng);
/* Runs the engine's work on `stream` (a hipStream_t; NULL is the device's null stream). */
int hkhip_set_stream(hkhip_engine *eng, void *stream);
/* Returns the engine to the stream it created at init. */
int hkhip_use_own_stream(hkhip_engine *eng);
void *hkhip_stream(hkhip_engine *eng);
int hkhip_sync(hkhip_engine *eng);
const char *hkhip_last_error(void);
const char *hkhip_device_name(hkhip_engine *eng);

/* ---- capability and sizing (src/cuda/engine.zig:106-108 supports, abi_ops.zig:56-62) ---- */
int hkhip_supports(uint8_t t);
/* Bytes of rows x cols weights of type t in hk's file layout, or a negative error. */
int64_t hkhip_matrix_bytes(uint8_t t, uint32_t rows, uint32_t cols);
/* Bytes of the activation-quant buffer for n tokens of k values (both kinds). */
uint64_t hkhip_act_bytes(uint32_t n, uint32_t k);

/* ---- device memory (the thin shim over hipMalloc / hipMemcpyAsync, src/cuda.zig) ---- */
int hkhip_alloc(hkhip_engine *eng, uint64_t bytes, void **out);
void hkhip_dev_free(hkhip_engine *eng, void *p);
int hkhip_copy_h2d(hkhip_engine *eng, void *dst, const void *src, uint64_t bytes);
int hkhip_copy_d2h(hkhip_engine *eng, void *dst, const void *src, uint64_t bytes);

/* ---- weights (Engine.upload, src/cuda/engine.zig:493-506) ----
 * Copies `bytes` of hk-file-layout weights from `src` (host memory, e.g. the mmap'd .hk
 * tensor, or device memory when src_on_device != 0) to the device and repacks them into the
 * device layout. Refuses cols % 32 != 0 or cols not a whole number of blocks
 * (UNSUPPORTED_SHAPE), unknown types (UNSUPPORTED_TYPE) and bytes != matrix_bytes. */
int hkhip_upload(hkhip_engine *eng, const void *src, uint64_t bytes, uint8_t t, uint32_t rows,
                 uint32_t cols, int src_on_device, hkhip_mat *out);
void hkhip_free(hkhip_engine *eng, hkhip_mat *m);

/* Decodes rows [row0, row0 + nrows) of a device matrix to f32 [nrows][cols] in device memory,
 * bit-for-bit as dequantizeRow (src/quant/dequant.zig:550-591). */
int hkhip_dequantize(hkhip_engine *eng, const hkhip_mat *m, uint32_t row0, uint32_t nrows, float *out_dev);

/* ---- activations (prepare: src/cuda/engine.zig:614-630; CPU arithmetic vecdot.zig:134-180) ----
 * Quantizes x_dev [n][k] f32 into xq_dev (hkhip_act_bytes(n, k) bytes) as `kind`. The buffer
 * holds both kinds side by side, so one input prepared once serves every product reading it. */
int hkhip_qact(hkhip_engine *eng, const float *x_dev, uint32_t n, uint32_t k, int kind, void *xq_dev);
/* Reads one kind back in hk's block structs: A8 as {f32 d, i32 s, i8 qs[32]} (40 B) per 32,
 * Q8K as {f32 d, i8 qs[256], i16 bsums[16]} (292 B) per 256 (vecdot.zig:22-26, blocks.zig:25). */
int hkhip_act_export(hkhip_engine *eng, const void *xq_dev, uint32_t n, uint32_t k, int kind, void *host_out);

/* ---- products (mm: src/cuda/engine.zig:581-611) ----
 * y_dev[t][r] (=|+=) dot(W[r], x[t]) + bias[r] for t < n, from activations already prepared
 * with hkhip_qact for the matrix's kind (A8: Q8_0, IQ4_NL; Q8K: Q4_K, Q6_K). bias may be NULL.
 * hkhip_matvec: decode kernels, 1 <= n <= 8 (src/kernels_impl.zig:14-33 rows).
 * hkhip_gemm:   prefill MFMA kernels, any n >= 1 (src/quant/gemm.zig tiles).
 * hkhip_mm:     picks matvec for n <= 8, then 8-token matvec passes up to the GEMM's break-even
 *               (Q6_K / Q8_0: 32 tokens, IQ4_NL: 24; Q4_K has none), then gemm (the CPU engine's
 *               switch is matmul.zig:18 min_tiled_tokens = 8).
 * mode is HKHIP_STORE, HKHIP_ACCUMULATE or HKHIP_SILU_MUL. */
int hkhip_matvec(hkhip_engine *eng, const hkhip_mat *m, const void *xq_dev, float *y_dev, uint32_t n,
                 const float *bias_dev, int mode);
int hkhip_gemm(hkhip_engine *eng, const hkhip_mat *m, const void *xq_dev, float *y_dev, uint32_t n,
               const float *bias_dev, int mode);
int hkhip_mm(hkhip_engine *eng, const hkhip_mat *m, const void *xq_dev, float *y_dev, uint32_t n,
             const float *bias_dev, int mode);

/* Fused decode products: up to 4 matrices that read the same input (q/k/v; gate/up) in one
 * launch, as matmul.runParts fuses them on the CPU (src/engine/matmul.zig:96-144). All parts
 * share type and cols. Give the input either as f32 x_dev [n][cols], which the kernel quantizes
 * itself with the qact arithmetic (no separate hkhip_qact launch), or as xq_dev prepared by
 * hkhip_qact (x_dev NULL). ys[i] / biases[i] belong to mats[i]; biases may be NULL or hold
 * NULLs. 1 <= n <= 8. */
int hkhip_matvec_parts(hkhip_engine *eng, const hkhip_mat *mats, uint32_t nparts, const float *x_dev,
                       const void *xq_dev, uint32_t n, float *const *ys, const float *const *biases, int mode);
/* The same on rmsnorm(x): each token's input is first scaled by 1 / sqrt(mean(x^2) + eps) and
 * multiplied by norm_dev [cols] (src/engine/ops.zig:10-29 rmsNorm), inside the products' own input
 * quantization -- the norm, prepare and runParts of cpu_backend.zig:264-271 in one launch. The
 * input must be f32; returns UNSUPPORTED_SHAPE for more than 8 tokens or rows too long for the
 * register decode kernel (the caller then normalizes separately). */
int hkhip_matvec_parts_rmsnorm(hkhip_engine *eng, const hkhip_mat *mats, uint32_t nparts, const float *x_dev,
                               const float *norm_dev, float eps, uint32_t n, float *const *ys,
                               const float *const *biases, int mode);

/* ---- product without allocation (no counterpart in the reference) ----
 * For callers that cannot allocate device memory: code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc. Same result as hkhip_qact(x_dev -> xq) followed by
 * hkhip_mm(m, xq, ...), bit for bit, but the activation buffer is a fixed device array inside the
 * library (HKHIP_NOALLOC_SCRATCH_BYTES per device, held until the process ends), so the call
 * allocates nothing. Refuses (UNSUPPORTED_SHAPE) inputs whose buffer, hkhip_act_bytes(n, cols),
 * exceeds that size: e.g. 512 tokens at cols 14336 (19.4 MiB) fit, 1024 tokens there do not.
 * All calls on one device share the buffer: calls that overlap in time on one device (two
 * streams, two threads) race, so serialise them. */
#define HKHIP_NOALLOC_SCRATCH_BYTES (24ull << 20)
int hkhip_mm_noalloc(hkhip_engine *eng, const hkhip_mat *m, const float *x_dev, float *y_dev, uint32_t n,
                     const float *bias_dev, int mode);

/* ---- whole network (the device engine: src/cuda/engine.zig Engine, driven through the seam
 * src/backend/backend.zig:128-209 Device: forward(items), forwardPartial, logits(indices), release,
 * maxRows, layerCount, isPartial; sized by bytesNeeded / layerBytes, engine.zig:155-190) ----
 * A decoder of n_layers blocks, each
 *   xb = rmsnorm(x) * attn_norm; q, k, v = Wq xb + bq, Wk xb + bk, Wv xb + bv;
 *   q, k = rope(headnorm(q, q_norm), headnorm(k, k_norm)); K/V cache (f16) += k, v at the position;
 *   att = causal GQA attention softmax(q K^T / sqrt(head_dim)) V; x += Wo att;
 *   xb = rmsnorm(x) * ffn_norm; x += Wdown (silu(Wgate xb) * (Wup xb)),
 * between an embedding lookup (a row of tok_embd, decoded) and logits = Woutput (rmsnorm(x) *
 * out_norm) (the CPU engine's order, src/engine/cpu_backend.zig:248-331).
 * A pass runs the tokens of one or more sequences (items); each sequence has its own K/V cache slot
 * of max_ctx positions, assigned on the sequence's first item (engine.zig:556-568 slotFor) and freed
 * by hkhip_net_release. Passes of up to 8 tokens run the decode kernels (RMS norm fused into the
 * products' input quantization, residual adds as accumulate-mode products, gate/up as one
 * silu(gate)*up launch; from 5 tokens the Q4_K / Q6_K products go through the fused quantizer and
 * the small-batch MFMA kernel; one-token passes do the q/k norms, RoPE and cache writes inside the
 * attention kernel) and are captured in a HIP graph per (token count, attention chunk count) after
 * their first run: tokens, positions and slots are read from device memory. Longer passes run the
 * MFMA GEMMs; their attention runs each sequence's consecutive run of positions longer than 8 on
 * the f16 MFMA prefill kernel, the other items on the decode attention kernel.
 * Matrices are hk file-layout bytes in host memory, copied at load; Wgate and Wup must share their
 * type; Wq, Wk and Wv that share theirs run as one product over their stacked rows (else as three,
 * e.g. a Q6_K Wv beside Q4_K Wq / Wk as in Q4_K_M files). Vectors (norms, biases) are f32 (HKHIP_F32). */
#define HKHIP_F32 0x00 /* hk StorageType f32 (src/format.zig:28) */
/* More error codes of the engine (src/cuda/engine.zig:31-40). */
#define HKHIP_E_NO_SLOT -7       /* NoGpuSlot: every cache slot is held by another sequence */
#define HKHIP_E_CONTEXT_FULL -8  /* ContextFull: an item's position is >= max_ctx */
#define HKHIP_E_PARTIAL -9       /* PartialEngine: forward on a partial network (or forward_partial on a full one) */
typedef struct hkhip_net hkhip_net;
typedef struct hkhip_net_config {
    uint32_t dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, vocab;
    uint32_t rope_dim;  /* rotated dimensions of a head (head_dim for full rotary) */
    uint32_t rope_neox; /* 0: pairs (2i, 2i+1) ("norm" style); 1: pairs (i, i + rope_dim/2) */
    uint32_t max_ctx;   /* K/V cache positions per sequence (Options.n_ctx) */
    float rms_eps, rope_base;
    /* RoPE as hk's model setup computes it for its device engines (src/engine/model.zig:123-124,
     * ops.zig ropeInvFreq / ropeMscale; src/cuda/engine.zig takes both at init): rope_dim / 2
     * inverse frequencies in host memory, read at create (NULL: rope_base^(-2i/rope_dim), no
     * scaling), and the multiplier of every cos and sin (0: 1; yarn scaling sets it). */
    const float *inv_freq;
    float rope_mscale;
} hkhip_net_config;
/* src/cuda/engine.zig:43-58 Options. */
typedef struct hkhip_net_options {
    uint32_t slots;   /* sequences that can hold a cache at once (0: 1) */
    uint32_t layers;  /* leading layers on the device; 0 or >= n_layers: all. Fewer: a partial network
                       * (no embedding, final norm or output; hkhip_net_forward_partial only) */
    uint32_t n_batch; /* most tokens in one pass; buffers are sized for it at create (0: grown on demand) */
    /* Test knob (as the CUDA engine's slice_positions, engine.zig:268): most decode attention
     * chunks merged inside the attention launch; more go through the separate merge kernel (0: 256). */
    uint32_t attn_merge_max;
    /* Decode attention kernel (a tuning knob, results equal to rounding): 0 chooses by size (the
     * grouped kernel, one workgroup per key/value head serving its query heads on the MFMA units,
     * once the per-head kernel would need more waves than the GPU runs at once); 1 the grouped
     * kernel whenever the head dim allows it (64 or 128); 2 the per-head kernel. */
    uint32_t attn_gqa;
} hkhip_net_options;
/* A tensor in hk's file layout in host memory; data NULL for an absent optional tensor. */
typedef struct hkhip_net_tensor {
    const void *data;
    uint64_t bytes;
    uint8_t t;
} hkhip_net_tensor;
typedef struct hkhip_net_layer {
    hkhip_net_tensor attn_norm, wq, wk, wv, bq, bk, bv, q_norm, k_norm, wo, ffn_norm, w_gate, w_up, w_down;
} hkhip_net_layer;
/* One token of one sequence in a pass (src/engine/kv.zig:22-29 Item). seq identifies the sequence
 * (hk passes its KvCache's address); items of one sequence appear in increasing position order. */
typedef struct hkhip_item {
    uint64_t seq;
    uint32_t token;
    uint32_t pos;
} hkhip_item;
/* Engine.init (engine.zig:276-...): caches for opts->slots sequences of cfg->max_ctx positions over
 * the device layers. hkhip_net_create is the same with default options (one slot, every layer,
 * buffers grown on demand). */
int hkhip_net_create_opts(hkhip_engine *eng, const hkhip_net_config *cfg, const hkhip_net_options *opts,
                          hkhip_net **out);
int hkhip_net_create(hkhip_engine *eng, const hkhip_net_config *cfg, hkhip_net **out);
void hkhip_net_destroy(hkhip_net *net);
/* Layers at or past the device layer count are refused (a partial network holds only its own). */
int hkhip_net_load_layer(hkhip_net *net, uint32_t layer, const hkhip_net_layer *l);
/* Not for partial networks (they have no embedding or output). */
int hkhip_net_load_io(hkhip_net *net, hkhip_net_tensor tok_embd, hkhip_net_tensor out_norm, hkhip_net_tensor output);
/* Device.forward (engine.zig:706-710): one pass over items[0..n) of one or more sequences; each
 * item's key and value go to its sequence's slot, and every item attends to positions 0..pos of its
 * own sequence (the items before it in the same pass included). Keeps every item's final hidden
 * state for hkhip_net_logits_rows. Errors: NO_SLOT, CONTEXT_FULL, PARTIAL, BAD_ARGUMENT (token >=
 * vocab, positions of a sequence not increasing, n > n_batch). Returns when the pass is done. */
int hkhip_net_forward_items(hkhip_net *net, const hkhip_item *items, uint32_t n);
/* Device.forwardPartial (engine.zig:716-721): a partial network's pass over items whose embedded
 * hidden states hidden_host [n][dim] (host memory) the caller made; on return hidden_host holds the
 * state after the last device layer. */
int hkhip_net_forward_partial(hkhip_net *net, const hkhip_item *items, uint32_t n, float *hidden_host);
/* Device.logits (engine.zig:799-817): logits of the given items of the last pass, one vocab row each
 * in the order of idx, to host_out [n][vocab]; 1 <= n <= hkhip_net_max_rows. One pass over the
 * output matrix for all rows. */
int hkhip_net_logits_rows(hkhip_net *net, const uint32_t *idx, uint32_t n, float *host_out);
/* Device.logits as the reference returns it (engine.zig:799-816: a slice of the engine's own host
 * buffer, valid until the next call): the same rows, in pinned host memory the network owns
 * ([max_rows][vocab] floats, allocated on the first call); *rows points at them until the next
 * call on net. No copy into the caller's memory. */
int hkhip_net_logits_view(hkhip_net *net, const uint32_t *idx, uint32_t n, const float **rows);
/* Device.release (engine.zig:570-575): frees the slot of sequence seq (nothing if it holds none). */
void hkhip_net_release(hkhip_net *net, uint64_t seq);
/* Device.maxRows / layerCount / isPartial (backend.zig:147-185). */
uint32_t hkhip_net_max_rows(const hkhip_net *net);
uint32_t hkhip_net_layer_count(const hkhip_net *net);
int hkhip_net_is_partial(const hkhip_net *net);
/* Runs tokens[0..n) of slot 0's sequence (seq 0) at positions pos0.. and computes the last token's
 * logits inside the pass (read with hkhip_net_logits / hkhip_net_logits_dev). */
int hkhip_net_forward(hkhip_net *net, const uint32_t *tokens, uint32_t n, uint32_t pos0);
/* Logits of the last token of the last hkhip_net_forward: vocab floats, to host memory. */
int hkhip_net_logits(hkhip_net *net, float *host_out);
/* The logits buffer in device memory (the last forward's, or the last logits_rows' rows; valid
 * until the next call). */
const float *hkhip_net_logits_dev(hkhip_net *net);
/* bytesNeeded / layerBytes (engine.zig:155-190), the planner's estimate (backend.zig:92-126
 * probeCuda): device bytes a network of cfg / opts would allocate for these tensors (only their
 * bytes and types are read; layers holds cfg->n_layers entries), plus a 64 MiB margin for the
 * runtime, and the device bytes of one layer's tensors. Both count the device layouts (stacked
 * q/k/v, interleaved gate/up, split planes), the caches (keys, values and the transposed values
 * the prefill attention reads) and the pass buffers for max(n_batch, 8) tokens (64 when n_batch
 * is 0). max_ctx may be 0 (the planner's base: bytes at n_ctx 0, then the per-position step from
 * n_ctx 1). 0 on a bad argument. hkhip_net_device_bytes: what a network holds now (bytes_needed without the margin,
 * once every tensor is loaded and with n_batch set). */
#define HKHIP_NET_MARGIN_BYTES (64ull << 20)
uint64_t hkhip_net_bytes_needed(const hkhip_net_config *cfg, const hkhip_net_options *opts,
                                const hkhip_net_layer *layers, hkhip_net_tensor tok_embd, hkhip_net_tensor out_norm,
                                hkhip_net_tensor output);
uint64_t hkhip_net_layer_bytes(const hkhip_net_config *cfg, const hkhip_net_layer *l);
uint64_t hkhip_net_device_bytes(const hkhip_net *net);

/* ---- host-pointer products (secondary boundary: src/c_api.zig:1380-1400, hk.h:451-453,
 * src/engine/abi_ops.zig:65-107) ----
 * y[t*m + r] = dot(W[r], x[t]) + bias[r] with W, x, bias, y in host memory, on the process's
 * default engine (device 0). On failure y is filled with NaN and a negative code returned. */
int hkhip_gemm_host(uint8_t t, const void *w, const float *x, const float *bias, float *y, uint64_t m,
                    uint64_t k, uint64_t n);
int hkhip_gemv_q8_0(const void *w, const float *x, const float *bias, float *y, uint64_t m, uint64_t k);
int hkhip_gemv_q4_0(const void *w, const float *x, const float *bias, float *y, uint64_t m, uint64_t k); /* hk.h:452 */
int hkhip_gemv_q4_k(const void *w, const float *x, const float *bias, float *y, uint64_t m, uint64_t k);
int hkhip_gemv_q6_k(const void *w, const float *x, const float *bias, float *y, uint64_t m, uint64_t k);
int hkhip_gemv_iq4_nl(const void *w, const float *x, const float *bias, float *y, uint64_t m, uint64_t k);

#ifdef __cplusplus
}
#endif
#endif /* HKHIP_H */
