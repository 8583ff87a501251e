// The C ABI of include/hkhip.h: engine lifetime, weight upload, activation prepare and the
// product dispatch. Host code only; the kernels live in weights.hip, qact.hip, mmvq.hip, mm.hip.
//
// Reference behaviour mirrored here:
//   upload validation       src/cuda/engine.zig:493-506 (cols % 32, whole blocks)
//   kernel choice by tokens src/engine/matmul.zig:18,107 (n >= 8 -> batch kernel)
//   matrixBytes             src/engine/abi_ops.zig:56-62
//   host gemm / gemv + NaN  src/engine/abi_ops.zig:65-107, src/c_api.zig:16-18,1380-1400
#include <mutex>
#include <stdio.h>
#include <stdarg.h>
#include <string.h>
#include <math.h>

#include "common.hpp"

using namespace hkhip;

static thread_local char g_err[512] = "";

// Activation buffer of hkhip_mm_noalloc: a file-scope device array, so that entry point needs no
// allocation. Every device holds its own copy until the process ends. Host code never passes the
// array's name to a kernel or a copy (on the host it is only a stand-in for the symbol): it uses
// the per-device address that hkhip_init looks up with hipGetSymbolAddress.
static __device__ __align__(256) uint8_t scratch[HKHIP_NOALLOC_SCRATCH_BYTES];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices] = {};

static int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hkhip::set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

static int hip_fail(hipError_t e, const char *what) {
    int code = e == hipErrorOutOfMemory ? HKHIP_E_OUT_OF_DEVICE_MEMORY : HKHIP_E_DEVICE_FAILED;
    return fail(code, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                     \
    do {                                        \
        hipError_t e_ = (expr);                 \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

static int enter(hkhip_engine *eng) {
    if (!eng) return fail(HKHIP_E_BAD_ARGUMENT, "null engine");
    HIP_TRY(hipSetDevice(eng->device), "hipSetDevice");
    return HKHIP_OK;
}

extern "C" {

const char *hkhip_last_error(void) { return g_err; }

int hkhip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int hkhip_init(int device, hkhip_engine **out) {
    if (!out) return fail(HKHIP_E_BAD_ARGUMENT, "null out");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(HKHIP_E_NO_DEVICE, "no HIP device found");
    if (device < 0 || device >= n) return fail(HKHIP_E_NO_DEVICE, "device %d out of range (%d devices)", device, n);
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    hipDeviceProp_t p;
    HIP_TRY(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties");
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(HKHIP_E_NO_DEVICE, "device %d is %s; the kernels are built for gfx950", device, p.gcnArchName);
    if (device >= kMaxDevices) return fail(HKHIP_E_NO_DEVICE, "device %d: at most %d devices", device, kMaxDevices);
    {
        // Once per device, with that device current: the address of this device's copy of the
        // no-allocation entry point's activation buffer.
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (!g_scratch_ptr[device]) {
            void *ptr = nullptr;
            HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
            g_scratch_ptr[device] = ptr;
        }
    }
    hkhip_engine *e = new hkhip_engine();
    e->device = device;
    hipError_t err = hipStreamCreateWithFlags(&e->own, hipStreamNonBlocking);
    if (err != hipSuccess) {
        delete e;
        return hip_fail(err, "hipStreamCreate");
    }
    e->cur = e->own;
    snprintf(e->name, sizeof e->name, "%s (%s)", p.name, p.gcnArchName);
    *out = e;
    return HKHIP_OK;
}

void hkhip_destroy(hkhip_engine *eng) {
    if (!eng) return;
    (void)hipSetDevice(eng->device);
    (void)hipStreamSynchronize(eng->cur);
    (void)hipStreamDestroy(eng->own);
    delete eng;
}

int hkhip_set_stream(hkhip_engine *eng, void *stream) {
    int rc = enter(eng);
    if (rc) return rc;
    eng->cur = reinterpret_cast<hipStream_t>(stream);
    return HKHIP_OK;
}

int hkhip_use_own_stream(hkhip_engine *eng) {
    int rc = enter(eng);
    if (rc) return rc;
    eng->cur = eng->own;
    return HKHIP_OK;
}

void *hkhip_stream(hkhip_engine *eng) { return eng ? reinterpret_cast<void *>(eng->cur) : nullptr; }

const char *hkhip_device_name(hkhip_engine *eng) { return eng ? eng->name : ""; }

int hkhip_sync(hkhip_engine *eng) {
    int rc = enter(eng);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize(eng->cur), "hipStreamSynchronize");
    return HKHIP_OK;
}

int hkhip_supports(uint8_t t) { return block_elems(t) != 0; }

int64_t hkhip_matrix_bytes(uint8_t t, uint32_t rows, uint32_t cols) {
    const int el = block_elems(t);
    if (!el) return fail(HKHIP_E_UNSUPPORTED_TYPE, "storage type 0x%02x has no HIP kernel", t);
    if (cols % el) return fail(HKHIP_E_UNSUPPORTED_SHAPE, "cols %u is not a whole number of %d-weight blocks", cols, el);
    return int64_t(rows) * (cols / el) * block_bytes(t);
}

uint64_t hkhip_act_bytes(uint32_t n, uint32_t k) { return act_layout(n, k).total; }

int hkhip_alloc(hkhip_engine *eng, uint64_t bytes, void **out) {
    int rc = enter(eng);
    if (rc) return rc;
    if (!out) return fail(HKHIP_E_BAD_ARGUMENT, "null out");
    *out = nullptr;
    HIP_TRY(hipMalloc(out, bytes ? bytes : 1), "hipMalloc");
    return HKHIP_OK;
}

void hkhip_dev_free(hkhip_engine *eng, void *p) {
    if (!eng || !p) return;
    (void)hipSetDevice(eng->device);
    (void)hipFree(p);
}

int hkhip_copy_h2d(hkhip_engine *eng, void *dst, const void *src, uint64_t bytes) {
    int rc = enter(eng);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, eng->cur), "hipMemcpyAsync H2D");
    HIP_TRY(hipStreamSynchronize(eng->cur), "hipStreamSynchronize");
    return HKHIP_OK;
}

int hkhip_copy_d2h(hkhip_engine *eng, void *dst, const void *src, uint64_t bytes) {
    int rc = enter(eng);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, eng->cur), "hipMemcpyAsync D2H");
    HIP_TRY(hipStreamSynchronize(eng->cur), "hipStreamSynchronize");
    return HKHIP_OK;
}

static int check_shape(uint8_t t, uint32_t cols) {
    const int el = block_elems(t);
    if (!el) return fail(HKHIP_E_UNSUPPORTED_TYPE, "storage type 0x%02x has no HIP kernel", t);
    // The kernels read weights and activations in blocks of 32 and whole blocks per row.
    if (cols == 0 || cols % 32 || cols % el)
        return fail(HKHIP_E_UNSUPPORTED_SHAPE, "cols %u must be a positive multiple of 32 and of %d", cols, el);
    return HKHIP_OK;
}

int hkhip_upload(hkhip_engine *eng, const void *src, uint64_t bytes, uint8_t t, uint32_t rows, uint32_t cols,
                 int src_on_device, hkhip_mat *out) {
    int rc = enter(eng);
    if (rc) return rc;
    if (!out) return fail(HKHIP_E_BAD_ARGUMENT, "null out");
    memset(out, 0, sizeof *out);
    if ((rc = check_shape(t, cols))) return rc;
    const uint64_t need = uint64_t(rows) * (cols / block_elems(t)) * block_bytes(t);
    if (bytes != need) return fail(HKHIP_E_BAD_ARGUMENT, "got %llu bytes, %ux%u of type 0x%02x needs %llu",
                                   (unsigned long long)bytes, rows, cols, t, (unsigned long long)need);
    if (!src && need) return fail(HKHIP_E_BAD_ARGUMENT, "null source");
    WLayout L = weight_layout(t, rows, cols);
    void *mem = nullptr;
    HIP_TRY(hipMalloc(&mem, L.total ? L.total : 1), "hipMalloc weights");
    hipError_t e = hipSuccess;
    if (t == HKHIP_Q4_K || t == HKHIP_Q5_K || fallback_type(t)) { // device layout = file layout
        e = hipMemcpyAsync(mem, src, need, src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, eng->cur);
    } else {
        const uint8_t *staged = reinterpret_cast<const uint8_t *>(src);
        void *tmp = nullptr;
        if (!src_on_device && need) {
            e = hipMalloc(&tmp, need);
            if (e == hipSuccess) e = hipMemcpyAsync(tmp, src, need, hipMemcpyHostToDevice, eng->cur);
            staged = reinterpret_cast<const uint8_t *>(tmp);
        }
        if (e == hipSuccess) e = launch_repack(t, staged, reinterpret_cast<uint8_t *>(mem), rows, cols, eng->cur);
        if (e == hipSuccess) e = hipStreamSynchronize(eng->cur);
        if (tmp) (void)hipFree(tmp);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(eng->cur);
    if (e != hipSuccess) {
        (void)hipFree(mem);
        return hip_fail(e, "upload");
    }
    out->mem = mem;
    out->file_bytes = need;
    out->dev_bytes = L.total;
    out->rows = rows;
    out->cols = cols;
    out->t = t;
    out->owned = 1;
    return HKHIP_OK;
}

void hkhip_free(hkhip_engine *eng, hkhip_mat *m) {
    if (!eng || !m || !m->mem) return;
    (void)hipSetDevice(eng->device);
    if (m->owned) (void)hipFree(m->mem);
    m->mem = nullptr;
}

static int check_mat(const hkhip_mat *m) {
    if (!m || !m->mem) return fail(HKHIP_E_BAD_ARGUMENT, "null matrix");
    return check_shape(m->t, m->cols);
}

int hkhip_dequantize(hkhip_engine *eng, const hkhip_mat *m, uint32_t row0, uint32_t nrows, float *out_dev) {
    int rc = enter(eng);
    if (rc || (rc = check_mat(m))) return rc;
    if (uint64_t(row0) + nrows > m->rows) return fail(HKHIP_E_BAD_ARGUMENT, "rows [%u, %u) outside %u", row0, row0 + nrows, m->rows);
    if (nrows && !out_dev) return fail(HKHIP_E_BAD_ARGUMENT, "null output");
    HIP_TRY(launch_dequant(m->t, reinterpret_cast<const uint8_t *>(m->mem), m->rows, m->cols, row0, nrows, out_dev,
                           eng->cur), "dequant launch");
    return HKHIP_OK;
}

int hkhip_qact(hkhip_engine *eng, const float *x_dev, uint32_t n, uint32_t k, int kind, void *xq_dev) {
    int rc = enter(eng);
    if (rc) return rc;
    if (kind != HKHIP_ACT_A8 && kind != HKHIP_ACT_Q8K) return fail(HKHIP_E_BAD_ARGUMENT, "unknown activation kind %d", kind);
    if (k == 0 || k % 32) return fail(HKHIP_E_UNSUPPORTED_SHAPE, "k %u is not a positive multiple of 32", k);
    if (kind == HKHIP_ACT_Q8K && k % QK_K) return fail(HKHIP_E_UNSUPPORTED_SHAPE, "Q8K needs k %% 256 == 0, got %u", k);
    if (n && (!x_dev || !xq_dev)) return fail(HKHIP_E_BAD_ARGUMENT, "null buffer");
    HIP_TRY(launch_qact(x_dev, n, k, kind, reinterpret_cast<uint8_t *>(xq_dev), eng->cur), "qact launch");
    return HKHIP_OK;
}

int hkhip_act_export(hkhip_engine *eng, const void *xq_dev, uint32_t n, uint32_t k, int kind, void *host_out) {
    int rc = enter(eng);
    if (rc) return rc;
    if (kind != HKHIP_ACT_A8 && kind != HKHIP_ACT_Q8K) return fail(HKHIP_E_BAD_ARGUMENT, "unknown activation kind %d", kind);
    if (k == 0 || k % (kind == HKHIP_ACT_A8 ? 32 : QK_K)) return fail(HKHIP_E_UNSUPPORTED_SHAPE, "bad k %u", k);
    const uint64_t nb = uint64_t(n) * k / (kind == HKHIP_ACT_A8 ? 32 : QK_K);
    const uint64_t bytes = nb * (kind == HKHIP_ACT_A8 ? 40 : 292);
    if (!nb) return HKHIP_OK;
    void *tmp = nullptr;
    HIP_TRY(hipMalloc(&tmp, bytes), "hipMalloc");
    hipError_t e = launch_act_pack(reinterpret_cast<const uint8_t *>(xq_dev), n, k, kind, reinterpret_cast<uint8_t *>(tmp), eng->cur);
    if (e == hipSuccess) e = hipMemcpyAsync(host_out, tmp, bytes, hipMemcpyDeviceToHost, eng->cur);
    if (e == hipSuccess) e = hipStreamSynchronize(eng->cur);
    (void)hipFree(tmp);
    if (e != hipSuccess) return hip_fail(e, "act export");
    return HKHIP_OK;
}

static int check_product(const hkhip_mat *m, const void *xq, float *y, uint32_t n, int mode) {
    int rc = check_mat(m);
    if (rc) return rc;
    if (mode != HKHIP_STORE && mode != HKHIP_ACCUMULATE && mode != HKHIP_SILU_MUL)
        return fail(HKHIP_E_BAD_ARGUMENT, "unknown mode %d", mode);
    if (mode == HKHIP_SILU_MUL && m->rows % 2)
        return fail(HKHIP_E_BAD_ARGUMENT, "silu(gate)*up needs interleaved gate/up rows (an even count)");
    if ((act_kind(m->t) == HKHIP_ACT_Q8K || fallback_type(m->t)) && m->cols % QK_K)
        return fail(HKHIP_E_UNSUPPORTED_SHAPE, "cols %u: the products of this type take whole 256-value groups", m->cols);
    if (n && (!xq || !y)) return fail(HKHIP_E_BAD_ARGUMENT, "null buffer");
    return HKHIP_OK;
}

// NVFP4 is dotted against the f32 input itself (vecdot.zig:189): no prepared buffer holds it.
static int check_prepared(const hkhip_mat *m) {
    if (act_kind(m->t) == HKHIP_ACT_F32)
        return fail(HKHIP_E_UNSUPPORTED_TYPE, "type 0x%02x takes an f32 input: use hkhip_matvec_parts with x, "
                                              "hkhip_mm_noalloc or hkhip_gemm_host", m->t);
    return HKHIP_OK;
}

int hkhip_matvec(hkhip_engine *eng, const hkhip_mat *m, const void *xq_dev, float *y_dev, uint32_t n,
                 const float *bias_dev, int mode) {
    int rc = enter(eng);
    if (rc || (rc = check_product(m, xq_dev, y_dev, n, mode)) || (rc = check_prepared(m))) return rc;
    if (n > 8) return fail(HKHIP_E_UNSUPPORTED_SHAPE, "matvec takes at most 8 tokens, got %u", n);
    if (mode == HKHIP_SILU_MUL && bias_dev) return fail(HKHIP_E_BAD_ARGUMENT, "silu(gate)*up takes no bias");
    if (n == 0) return HKHIP_OK;
    HIP_TRY(launch_mmvq(m->t, reinterpret_cast<const uint8_t *>(m->mem), m->rows, m->cols,
                        reinterpret_cast<const uint8_t *>(xq_dev), n, y_dev, bias_dev, mode, eng->cur), "mmvq launch");
    return HKHIP_OK;
}

int hkhip_matvec_parts(hkhip_engine *eng, const hkhip_mat *mats, uint32_t nparts, const float *x_dev,
                       const void *xq_dev, uint32_t n, float *const *ys, const float *const *biases, int mode) {
    int rc = enter(eng);
    if (rc) return rc;
    if (!mats || !ys || nparts < 1 || nparts > 4) return fail(HKHIP_E_BAD_ARGUMENT, "need 1..4 parts, got %u", nparts);
    if ((x_dev == nullptr) == (xq_dev == nullptr)) return fail(HKHIP_E_BAD_ARGUMENT, "give exactly one of x and xq");
    MvPartDesc parts[4];
    for (uint32_t i = 0; i < nparts; i++) {
        if ((rc = check_product(&mats[i], x_dev ? (const void *)x_dev : xq_dev, ys[i], n, mode))) return rc;
        if (mode == HKHIP_SILU_MUL && biases && biases[i])
            return fail(HKHIP_E_BAD_ARGUMENT, "silu(gate)*up takes no bias");
        if (mats[i].t != mats[0].t || mats[i].cols != mats[0].cols)
            return fail(HKHIP_E_BAD_ARGUMENT, "fused parts must share type and cols");
        parts[i] = MvPartDesc{reinterpret_cast<const uint8_t *>(mats[i].mem), ys[i], biases ? biases[i] : nullptr,
                              mats[i].rows};
    }
    if (n > 8) return fail(HKHIP_E_UNSUPPORTED_SHAPE, "matvec takes at most 8 tokens, got %u", n);
    if (n == 0) return HKHIP_OK;
    HIP_TRY(launch_mmvq_parts(mats[0].t, parts, int(nparts), mats[0].cols, x_dev,
                              reinterpret_cast<const uint8_t *>(xq_dev), n, mode, eng->cur), "mmvq launch");
    return HKHIP_OK;
}

int hkhip_matvec_parts_rmsnorm(hkhip_engine *eng, const hkhip_mat *mats, uint32_t nparts, const float *x_dev,
                               const float *norm_dev, float eps, uint32_t n, float *const *ys,
                               const float *const *biases, int mode) {
    int rc = enter(eng);
    if (rc) return rc;
    if (!mats || !ys || nparts < 1 || nparts > 4) return fail(HKHIP_E_BAD_ARGUMENT, "need 1..4 parts, got %u", nparts);
    if (!x_dev || !norm_dev) return fail(HKHIP_E_BAD_ARGUMENT, "null input or norm weights");
    MvPartDesc parts[4];
    for (uint32_t i = 0; i < nparts; i++) {
        if ((rc = check_product(&mats[i], x_dev, ys[i], n, mode))) return rc;
        if (mode == HKHIP_SILU_MUL && biases && biases[i])
            return fail(HKHIP_E_BAD_ARGUMENT, "silu(gate)*up takes no bias");
        if (mats[i].t != mats[0].t || mats[i].cols != mats[0].cols)
            return fail(HKHIP_E_BAD_ARGUMENT, "fused parts must share type and cols");
        parts[i] = MvPartDesc{reinterpret_cast<const uint8_t *>(mats[i].mem), ys[i], biases ? biases[i] : nullptr,
                              mats[i].rows};
    }
    if (n > 8) return fail(HKHIP_E_UNSUPPORTED_SHAPE, "the fused norm takes at most 8 tokens, got %u", n);
    if (n == 0) return HKHIP_OK;
    const hipError_t e = launch_mmvq_parts_norm(mats[0].t, parts, int(nparts), mats[0].cols, x_dev, nullptr, n, mode,
                                                norm_dev, eps, eng->cur);
    if (e == hipErrorNotSupported)
        return fail(HKHIP_E_UNSUPPORTED_SHAPE, "no fused-norm kernel for %u tokens of %u cols", n, mats[0].cols);
    HIP_TRY(e, "mmvq launch");
    return HKHIP_OK;
}

int hkhip_gemm(hkhip_engine *eng, const hkhip_mat *m, const void *xq_dev, float *y_dev, uint32_t n,
               const float *bias_dev, int mode) {
    int rc = enter(eng);
    if (rc || (rc = check_product(m, xq_dev, y_dev, n, mode)) || (rc = check_prepared(m))) return rc;
    if (mode == HKHIP_SILU_MUL && bias_dev) return fail(HKHIP_E_BAD_ARGUMENT, "silu(gate)*up takes no bias");
    if (n == 0) return HKHIP_OK;
    if ((n + 63) / 64 > 65535u) return fail(HKHIP_E_UNSUPPORTED_SHAPE, "too many tokens: %u", n);
    HIP_TRY(launch_mm(m->t, reinterpret_cast<const uint8_t *>(m->mem), m->rows, m->cols,
                      reinterpret_cast<const uint8_t *>(xq_dev), n, y_dev, bias_dev, mode, eng->cur), "mm launch");
    return HKHIP_OK;
}

// Fewest tokens for which the GEMM beats 8-token matvec passes (measured on MI355X at the
// Llama-3-8B FFN shapes: a GEMM pass costs about as much at 16 tokens as at 64, while each
// matvec pass of 8 tokens streams the weights once more).
static uint32_t gemm_min_tokens(int t, uint32_t rows) {
    switch (t) {
    case HKHIP_Q6_K:
    case HKHIP_Q8_0: return 33;
    case HKHIP_IQ4_NL: return 25;
    case HKHIP_Q5_K: case HKHIP_Q4_0: case HKHIP_Q4_1: case HKHIP_Q5_0: case HKHIP_Q5_1: case HKHIP_IQ4_XS:
        // Measured at 9-64 tokens: with 14336 rows the GEMM beats two decode passes from 9
        // tokens; with 4096 rows (K 14336) it costs 50-120 us at any count (Q4_1 50, IQ4_XS 66,
        // Q5_1 82, Q5_0 98, Q4_0 104, Q5_K 118), which the passes (20-25 us per 8 tokens) reach at
        // the counts below.
        if (rows >= 8192) return 9;
        return t == HKHIP_Q4_1 ? 17 : (t == HKHIP_IQ4_XS || t == HKHIP_Q5_1) ? 25 : t == HKHIP_Q5_0 ? 33 : 41;
    default: return 9;
    }
}

int hkhip_mm(hkhip_engine *eng, const hkhip_mat *m, const void *xq_dev, float *y_dev, uint32_t n,
             const float *bias_dev, int mode) {
    // The CPU engine tiles from min_tiled_tokens = 8 (matmul.zig:18); here the register matvec
    // covers up to 8 tokens and, below the GEMM's break-even, runs in passes of 8.
    if (n <= 8) return hkhip_matvec(eng, m, xq_dev, y_dev, n, bias_dev, mode);
    if (n >= gemm_min_tokens(m->t, m->rows)) return hkhip_gemm(eng, m, xq_dev, y_dev, n, bias_dev, mode);
    int rc = enter(eng);
    if (rc || (rc = check_product(m, xq_dev, y_dev, n, mode)) || (rc = check_prepared(m))) return rc;
    if (mode == HKHIP_SILU_MUL && bias_dev) return fail(HKHIP_E_BAD_ARGUMENT, "silu(gate)*up takes no bias");
    HIP_TRY(launch_mmvq(m->t, reinterpret_cast<const uint8_t *>(m->mem), m->rows, m->cols,
                        reinterpret_cast<const uint8_t *>(xq_dev), n, y_dev, bias_dev, mode, eng->cur), "mmvq launch");
    return HKHIP_OK;
}

int hkhip_mm_noalloc(hkhip_engine *eng, const hkhip_mat *m, const float *x_dev, float *y_dev, uint32_t n,
                     const float *bias_dev, int mode) {
    int rc = enter(eng);
    if (rc || (rc = check_product(m, x_dev, y_dev, n, mode))) return rc;
    if (n == 0) return HKHIP_OK;
    const uint64_t need = act_layout(n, m->cols).total;
    if (need > HKHIP_NOALLOC_SCRATCH_BYTES)
        return fail(HKHIP_E_UNSUPPORTED_SHAPE,
                    "hkhip_mm_noalloc: %u tokens x %u cols need %llu bytes of activation buffer, over its %llu",
                    n, m->cols, (unsigned long long)need, (unsigned long long)HKHIP_NOALLOC_SCRATCH_BYTES);
    if (act_kind(m->t) == HKHIP_ACT_F32) { // dotted against the f32 input: no buffer needed
        MvPartDesc p{reinterpret_cast<const uint8_t *>(m->mem), y_dev, bias_dev, m->rows};
        HIP_TRY(launch_fb_mv(m->t, &p, 1, m->cols, x_dev, nullptr, n, mode, eng->cur), "mmvq launch");
        return HKHIP_OK;
    }
    void *xq = g_scratch_ptr[eng->device]; // set by hkhip_init for this engine's device
    if (!xq) return fail(HKHIP_E_DEVICE_FAILED, "no activation buffer for device %d", eng->device);
    if ((rc = hkhip_qact(eng, x_dev, n, m->cols, act_kind(m->t), xq))) return rc;
    return hkhip_mm(eng, m, xq, y_dev, n, bias_dev, mode);
}

// ---- host-pointer products on a process-wide default engine ----

static std::mutex g_host_mu;
static hkhip_engine *g_host_eng = nullptr;

static void poison(float *y, uint64_t count) {
    if (!y) return;
    for (uint64_t i = 0; i < count; i++) y[i] = NAN;
}

int hkhip_gemm_host(uint8_t t, const void *w, const float *x, const float *bias, float *y, uint64_t m, uint64_t k,
                    uint64_t n) {
    std::lock_guard<std::mutex> lock(g_host_mu);
    const uint64_t ycount = m * n;
    int rc = HKHIP_OK;
    if (m > 0xffffffffu || k > 0xffffffffu || n > 0xffffffffu) rc = fail(HKHIP_E_UNSUPPORTED_SHAPE, "shape too large");
    if (!rc) rc = check_shape(t, uint32_t(k));
    if (!rc && act_kind(t) == HKHIP_ACT_Q8K && k % QK_K) rc = fail(HKHIP_E_UNSUPPORTED_SHAPE, "bad k");
    if (!rc && (!w || !x || !y)) rc = fail(HKHIP_E_BAD_ARGUMENT, "null pointer");
    if (rc) {
        poison(y, ycount);
        return rc;
    }
    if (m == 0 || n == 0) return HKHIP_OK;
    if (!g_host_eng && (rc = hkhip_init(0, &g_host_eng))) {
        poison(y, ycount);
        return rc;
    }
    hkhip_engine *eng = g_host_eng;
    hkhip_mat mat{};
    void *dx = nullptr, *dy = nullptr, *db = nullptr, *dq = nullptr;
    const uint64_t xbytes = n * k * 4, ybytes = ycount * 4;
    const int64_t wbytes = hkhip_matrix_bytes(t, uint32_t(m), uint32_t(k));
    rc = hkhip_upload(eng, w, uint64_t(wbytes), t, uint32_t(m), uint32_t(k), 0, &mat);
    if (!rc) rc = hkhip_alloc(eng, xbytes, &dx);
    if (!rc) rc = hkhip_alloc(eng, ybytes, &dy);
    if (!rc) rc = hkhip_alloc(eng, hkhip_act_bytes(uint32_t(n), uint32_t(k)), &dq);
    if (!rc && bias) rc = hkhip_alloc(eng, m * 4, &db);
    if (!rc) rc = hkhip_copy_h2d(eng, dx, x, xbytes);
    if (!rc && bias) rc = hkhip_copy_h2d(eng, db, bias, m * 4);
    if (act_kind(t) == HKHIP_ACT_F32) { // products on the f32 input itself, 8 tokens per pass
        for (uint64_t t0 = 0; !rc && t0 < n; t0 += 8) {
            const uint32_t nc = uint32_t(n - t0 < 8 ? n - t0 : 8);
            float *yc = reinterpret_cast<float *>(dy) + t0 * m;
            const float *bc = reinterpret_cast<float *>(db);
            rc = hkhip_matvec_parts(eng, &mat, 1, reinterpret_cast<float *>(dx) + t0 * k, nullptr, nc, &yc, &bc,
                                    HKHIP_STORE);
        }
    } else {
        if (!rc) rc = hkhip_qact(eng, reinterpret_cast<float *>(dx), uint32_t(n), uint32_t(k), act_kind(t), dq);
        if (!rc) rc = hkhip_mm(eng, &mat, dq, reinterpret_cast<float *>(dy), uint32_t(n), reinterpret_cast<float *>(db),
                               HKHIP_STORE);
    }
    if (!rc) rc = hkhip_copy_d2h(eng, y, dy, ybytes);
    hkhip_free(eng, &mat);
    hkhip_dev_free(eng, dx);
    hkhip_dev_free(eng, dy);
    hkhip_dev_free(eng, dq);
    hkhip_dev_free(eng, db);
    if (rc) poison(y, ycount);
    return rc;
}

int hkhip_gemv_q8_0(const void *w, const float *x, const float *bias, float *y, uint64_t m, uint64_t k) {
    return hkhip_gemm_host(HKHIP_Q8_0, w, x, bias, y, m, k, 1);
}
int hkhip_gemv_q4_0(const void *w, const float *x, const float *bias, float *y, uint64_t m, uint64_t k) {
    return hkhip_gemm_host(HKHIP_Q4_0, w, x, bias, y, m, k, 1);
}
int hkhip_gemv_q4_k(const void *w, const float *x, const float *bias, float *y, uint64_t m, uint64_t k) {
    return hkhip_gemm_host(HKHIP_Q4_K, w, x, bias, y, m, k, 1);
}
int hkhip_gemv_q6_k(const void *w, const float *x, const float *bias, float *y, uint64_t m, uint64_t k) {
    return hkhip_gemm_host(HKHIP_Q6_K, w, x, bias, y, m, k, 1);
}
int hkhip_gemv_iq4_nl(const void *w, const float *x, const float *bias, float *y, uint64_t m, uint64_t k) {
    return hkhip_gemm_host(HKHIP_IQ4_NL, w, x, bias, y, m, k, 1);
}

} // extern "C"
