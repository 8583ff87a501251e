// The whole-network device pass: embedding lookup, the decoder layers and the logits, on the
// quantized-linear kernels of this library plus the few kernels of this file (RMS norm, per-head
// norm + RoPE + K/V cache write, split-context attention and its combine, silu(gate)*up over
// interleaved rows).
//
// Reference behaviour mirrored (layer order and arithmetic of hk's engines):
//   layer order, residual adds         src/engine/cpu_backend.zig:248-322 forwardFrom
//   device pass and graph replay       src/cuda/engine.zig:646-797 runBatch / forwardImpl / runPass
//   rmsNorm / headNorm / swiglu        src/engine/ops.zig:10-38, 70-80
//   RoPE inverse frequencies, angles   src/engine/ops.zig:96-160 ropeInvFreq (no scaling) / ropeAngles
//   RoPE styles norm / neox            src/engine/ops.zig:164-185 ropeApply
//   attention (causal, GQA, 1/sqrt(hd), split slices merged by max/sum)
//                                      src/engine/attention.zig:44-133 run / merge
//   K/V cache in f16                   src/engine/kv.zig:1-11
//
// MI355X-specific choices: decode passes (1-8 tokens) fuse the RMS norm into the input staging of
// the q/k/v, gate/up and output products, make the residual adds accumulate-mode products, and
// use one silu(gate)*up launch over gate/up rows interleaved at load; the pass reads the tokens and
// positions from device memory, so one captured HIP graph per token count serves every position.
// Attention splits the context into fixed slices of ATT_SLICE positions (slices past a token's
// position only record an empty partial), so the launch shape never depends on the position.
#include <hip/hip_fp16.h>

#include <algorithm>
#include <map>
#include <math.h>
#include <string.h>
#include <vector>

#include "common.hpp"
#include "qact.hpp"
#include "quant.hpp"

using namespace hkhip;

namespace {

constexpr uint32_t ATT_SLICE = 64;      // positions per wave step of the decode attention
constexpr uint32_t MAX_DECODE = 8;      // tokens of a pass that runs the decode kernels (and a graph)
constexpr uint32_t ATT_MERGE_MAX = 256; // decode attention chunks the in-launch merge takes (more: attn_combine_kernel)
// Floats per decode attention chunk's {max, sum} pair, and 32-bit words per chunk counter: one
// 128-byte line each, since chunk workgroups on different XCDs write them through to the coherence
// point and writers sharing a line were measured to slow the pass (packed pairs: 1.664-1.670 vs
// 1.624-1.632 ms per Llama-3-8B token, 0.880-0.882 vs 0.806-0.830 per Qwen3-0.6B token; padded
// counters: 8 sequences per pass 2.839-2.870 vs 2.875-2.883 ms).
constexpr uint32_t ATT_ML = 32, ATT_CNT = 32;

// ---------------------------------------------------------------------------------------------
// Kernels
// ---------------------------------------------------------------------------------------------

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float block_sum(float v, float *red) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    const uint32_t w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = 0.0f;
    for (uint32_t i = 0; i < nw; i++) s += red[i];
    return s;
}

// out[t] = x[t] * (1 / sqrt(mean(x[t]^2) + eps)) * w, one workgroup per row (ops.zig:10-29).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                      float *__restrict__ out, uint32_t dim, float eps) {
    __shared__ float red[4];
    const float *xr = x + uint64_t(blockIdx.x) * dim;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) ss = fmaf(xr[i], xr[i], ss);
    ss = block_sum(ss, red);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, float(dim)) + eps));
    float *o = out + uint64_t(blockIdx.x) * dim;
    for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) o[i] = (xr[i] * inv) * w[i];
}

// One wave per (token, head): heads 0..nh-1 are query heads (normalized, rotated, written back),
// nh..nh+nkv-1 key heads (normalized, rotated, written to the f16 key cache), then nkv value heads
// (to the f16 value cache, and transposed to [kv head][hd][vt_stride] for the prefill attention).
// Token t sits at position pos[t] of the sequence whose caches are slot slot[t]. Cache layout
// [slot][layer][kv head][max_ctx][hd]; kc / vc / vt point at this layer of slot 0.
struct RopeArgs {
    float *q;
    const float *k, *v; // rows of the fused q/k/v output: stride sq (q) and skv (k, v) floats per token
    const float *q_norm, *k_norm; // [hd] or null
    const float *inv_freq;        // [rope_dim / 2]
    __half *kc, *vc;              // this layer's caches (slot 0)
    __half *vt;                   // this layer's transposed value cache [nkv][hd][vt_stride] (slot 0)
    const uint32_t *pos, *slot;   // per token
    uint64_t kv_slot, vt_slot;    // halves between slots of kc / vc and of vt
    uint32_t nh, nkv, hd, rope_half, neox, max_ctx, vt_stride, sq, skv;
    uint32_t nheads; // heads this launch covers: nh + nkv (keys), + nkv (values)
    float mscale;    // multiplier of every cos and sin (ops.zig ropeMscale)
    float eps;
    uint32_t ntok;   // tokens of the pass (the prefill launch's value rows)
};

// Four heads per workgroup, one per wave; each wave works on its own LDS row, so the waves never
// wait for each other (a wave's LDS accesses complete in order: only the compiler must keep them
// in order, which the wave barriers do).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
}
// One head row in a wave's LDS row h (hd values, lanes strided by 64): headNorm when nw is given
// (rmsNorm over the head, ops.zig:31-38), then ropeApply (ops.zig:171-185) with the angles' cos and
// sin from the table cst (rope_table). The fused decode attention kernels run the same steps on the
// rows they need (their sums over the head in other orders), so they agree to rounding.
__device__ __forceinline__ void head_norm_rope(float *h, const float *src, const float *nw, const float (*cst)[128],
                                               const RopeArgs &a, uint32_t lane) {
    const uint32_t hd = a.hd;
    for (uint32_t d = lane; d < hd; d += 64) h[d] = src[d];
    wave_sync();
    if (nw) {
        float ss = 0.0f;
        for (uint32_t d = lane; d < hd; d += 64) ss = fmaf(h[d], h[d], ss);
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, float(hd)) + a.eps));
        wave_sync();
        for (uint32_t d = lane; d < hd; d += 64) h[d] = (h[d] * inv) * nw[d];
        wave_sync();
    }
    for (uint32_t i = lane; i < a.rope_half; i += 64) {
        const float c = cst[0][i], s = cst[1][i];
        const uint32_t i0 = a.neox ? i : 2 * i, i1 = a.neox ? i + a.rope_half : 2 * i + 1;
        const float x0 = h[i0], x1 = h[i1];
        h[i0] = x0 * c - x1 * s;
        h[i1] = x0 * s + x1 * c;
    }
    wave_sync();
}

// cos and sin (times ropeMscale) of the rope_half rotation angles at position pos (ropeAngles,
// ops.zig:154-170) into cst, by the workgroup's threads; ends with a barrier.
__device__ __forceinline__ void rope_table(float (*cst)[128], uint32_t pos, const RopeArgs &a) {
    const float p = float(pos);
    for (uint32_t i = threadIdx.x; i < a.rope_half; i += blockDim.x) {
        float sn, cs;
        sincosf(p * a.inv_freq[i], &sn, &cs);
        cst[0][i] = cs * a.mscale;
        cst[1][i] = sn * a.mscale;
    }
    __syncthreads();
}

// Heads 4 bx .. 4 bx + 3 of token t (q, then k, then -- when a.nheads counts them -- v), one per
// wave: head norm and rotation (the angles' cos / sin computed once per workgroup: a quarter of
// the sines a wave each computed before) and the key and value rows into the caches. (One
// workgroup per token, its waves taking the heads in turn: Qwen3-0.6B's 512-token prefill 2.69-2.74
// vs 2.58-2.62 ms, a wave's heads one after another.)
__device__ __forceinline__ void rope_kv_block(const RopeArgs &a, uint32_t bx, uint32_t t) {
    const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t hh = 4 * bx + w;
    const uint32_t pos = a.pos[t];
    const uint64_t sl = a.slot[t];
    const uint32_t hd = a.hd;
    __shared__ float cst[2][128];
    __shared__ float hs[4][256];
    rope_table(cst, pos, a);
    if (hh >= a.nheads) return; // past the last head launched (whole wave; no workgroup barriers below)
    const bool isq = hh < a.nh, isk = !isq && hh < a.nh + a.nkv;
    if (!isq && !isk) { // value head: straight to the caches
        const uint32_t g = hh - a.nh - a.nkv;
        const float *src = a.v + uint64_t(t) * a.skv + g * hd;
        __half *dst = a.vc + sl * a.kv_slot + (uint64_t(g) * a.max_ctx + pos) * hd;
        __half *dt = a.vt + sl * a.vt_slot + uint64_t(g) * hd * a.vt_stride + pos;
        for (uint32_t d = lane; d < hd; d += 64) {
            const __half v = __float2half(src[d]);
            dst[d] = v;
            dt[uint64_t(d) * a.vt_stride] = v;
        }
        return;
    }
    const uint32_t g = isq ? hh : hh - a.nh;
    const float *src = isq ? a.q + uint64_t(t) * a.sq + g * hd : a.k + uint64_t(t) * a.skv + g * hd;
    float *h = hs[w];
    head_norm_rope(h, src, isq ? a.q_norm : a.k_norm, cst, a, lane);
    if (isq) {
        float *dst = a.q + uint64_t(t) * a.sq + g * hd;
        for (uint32_t d = lane; d < hd; d += 64) dst[d] = h[d];
    } else {
        __half *dst = a.kc + sl * a.kv_slot + (uint64_t(g) * a.max_ctx + pos) * hd;
        for (uint32_t d = lane; d < hd; d += 64) dst[d] = __float2half(h[d]);
    }
}

__global__ __launch_bounds__(256) void rope_kv_kernel(RopeArgs a) { rope_kv_block(a, blockIdx.x, blockIdx.y); }

// Value rows of a prefill pass to the f16 caches, 16 tokens of one key/value head per workgroup:
// the rows go to the value cache as they are and, through an LDS tile, to the transposed cache
// with consecutive lanes on consecutive tokens (consecutive positions within a sequence's run;
// decode passes write both in rope_kv_kernel).
__device__ __forceinline__ void v_cache_block(const RopeArgs &a, const float *__restrict__ v, uint32_t g, uint32_t ty) {
    __shared__ __half tile[16][258];
    __shared__ uint32_t tpos[16];
    __shared__ uint64_t tslot[16];
    const uint32_t t0 = ty * 16, tid = threadIdx.x, hd = a.hd, n = a.ntok;
    const uint32_t nt = n - t0 < 16 ? n - t0 : 16, kvd = a.skv; // row stride of v
    if (tid < nt) {
        tpos[tid] = a.pos[t0 + tid];
        tslot[tid] = a.slot[t0 + tid];
    }
    __syncthreads();
    for (uint32_t i = 4 * tid; i < nt * hd; i += 1024) { // hd is a multiple of 64: four values of one row
        const uint32_t tt = i / hd, d = i % hd;
        const float4 x = *reinterpret_cast<const float4 *>(v + uint64_t(t0 + tt) * kvd + g * hd + d);
        const __half h4[4] = {__float2half(x.x), __float2half(x.y), __float2half(x.z), __float2half(x.w)};
        __half *dst = a.vc + tslot[tt] * a.kv_slot + (uint64_t(g) * a.max_ctx + tpos[tt]) * hd + d;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            dst[k] = h4[k];
            tile[tt][d + k] = h4[k];
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < hd * 16; i += 256) {
        const uint32_t d = i / 16, tt = i % 16;
        if (tt < nt) a.vt[tslot[tt] * a.vt_slot + (uint64_t(g) * hd + d) * a.vt_stride + tpos[tt]] = tile[tt][d];
    }
}

// A prefill pass's rope / key writes (the first rx * n workgroups, as rope_kv_kernel's grid
// (rx, n)) and value writes (the rest, nkv x ceil(n / 16) workgroups of 16 tokens of one head) in one launch.
__global__ __launch_bounds__(256) void rope_kv_v_kernel(RopeArgs a, const float *__restrict__ v, uint32_t rx) {
    const uint32_t b = blockIdx.x, nr = rx * a.ntok;
    if (b < nr)
        rope_kv_block(a, b % rx, b / rx);
    else
        v_cache_block(a, v, (b - nr) % a.nkv, (b - nr) / a.nkv);
}

// Decode attention arguments (the kernel below): per (token, query head) the context of the
// token's own sequence, positions 0..pos[t] of slot slot[t].
struct AttnArgs {
    const float *q; // stride sq floats per token
    const __half *kc, *vc; // this layer of slot 0
    float *part; // chunk partials' sums (part_ml below)
    const uint32_t *pos, *slot;
    uint64_t kv_slot; // halves between slots
    uint32_t n, nh, nkv, hd, max_ctx;
    float scale;
    uint32_t sq;
    // Decode only. att: with one chunk per (head, token) the normalized result goes straight here
    // (part unused). fused (one-token passes): q is the projection's raw output, and the kernel
    // does rope_kv_kernel's work itself (the q and new key head norms and rotations, the new key
    // and value rows into the caches), with r's fields.
    float *att;
    int fused;
    RopeArgs r;
    // Several chunks: with cnt set, the last chunk workgroup of (head, token) to finish merges the
    // partials into merge_out itself (cnt: one counter per (token, head), zero between launches).
    uint32_t *cnt;
    float *merge_out;
    // The chunk partials: part holds the unnormalized sums [token][head][chunk][hd], part_ml the
    // {max, sum} pairs [token][head][chunk][ATT_ML].
    float *part_ml;
    // q8_on (grouped kernel, head blocks of whole 256-value blocks): the workgroup that writes a head
    // block's results also quantizes them into q8 (qact_q8k_kernel's planes for the pass's output
    // rows), for the o product's prepared input.
    int q8_on;
    Q8KOut q8;
};

// A lane's DL dimensions of one value row: DL halves in one (DL = 1: the low half) or two words.
template <int DL> struct VRow {
    uint32_t w[DL > 2 ? 2 : 1];
    __device__ float get(int j) const {
        const uint32_t b = DL == 1 ? w[0] : w[j >> 1] >> (16 * (j & 1));
        return __half2float(__ushort_as_half(uint16_t(b & 0xFFFFu)));
    }
    __device__ void load(const __half *p) {
        if constexpr (DL == 1)
            w[0] = *reinterpret_cast<const uint16_t *>(p);
        else if constexpr (DL == 2)
            w[0] = *reinterpret_cast<const uint32_t *>(p);
        else {
            const uint2 u = *reinterpret_cast<const uint2 *>(p);
            w[0] = u.x;
            w[1] = u.y;
        }
    }
    // Ties the loaded words to this point, so the compiler keeps the loads where they are issued
    // (ahead of every use) instead of sinking each next to its use.
    __device__ void pin() {
#pragma unroll
        for (int i = 0; i < (DL > 2 ? 2 : 1); i++) asm volatile("" : "+v"(w[i]));
    }
};

// Decode attention (passes of up to MAX_DECODE tokens): C chunk workgroups of NWV waves per (head
// block, token), C set by the context the pass reaches (host side: enough that every 64-position
// step up to the last position has a wave of its own; the context's loads spread over C times more
// CUs than one workgroup would use); wave w of chunk g takes step g*NWV + w. A head block
// is the G query heads that share one key/value head (the whole GQA group), so each key and value
// row is loaded once for all of them. A workgroup merges its waves' {max, sum, acc} per head in LDS
// (as the slice merge does, attention.zig:113-133) and writes the chunk's partials ({-inf, 0, 0...}
// past the token's position), which the last chunk to finish (or attn_combine_kernel) merges; with
// C = 1 it writes the normalized results itself. In a step a lane loads its position's key row
// (scores: lane = position, one dot per head against the heads' q rows in LDS), then the value rows
// go 16 bytes per lane: lane = (row r of the RPI rows one load covers, 8 dimensions), so a step is
// HD/8 + 64/RPI loads per lane whatever G is; the RPI partial sums of a dimension are added across
// lanes once, at the end.
//
// Passes whose tokens each have a slot of their own (every one-token pass) run fused: the raw q rows
// are normalized and rotated in the kernel (the same steps as rope_kv_kernel), and the wave whose
// step holds the token's position builds the new key
// row (norm, rotation, f16) and value row, uses them in place of the cache rows it loaded, and -- in
// the head block holding the group's first head -- writes them to the caches. The kernel follows
// the declarations below.

// Sum / max over a wave: DPP moves within each row of 16 lanes, then the four rows' results.
__device__ __forceinline__ float wave_sum_f(float v) {
    v += dpp_f<DPP_XOR1>(v);
    v += dpp_f<DPP_XOR2>(v);
    v += dpp_f<DPP_HALF_MIRROR>(v);
    v += dpp_f<DPP_MIRROR>(v);
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}
__device__ __forceinline__ float wave_max_f(float v) {
    const float r = row_max(v);
    return fmaxf(fmaxf(readlane_f(r, 0), readlane_f(r, 16)), fmaxf(readlane_f(r, 32), readlane_f(r, 48)));
}

// 16 bytes at p read at the device's coherence point, not from this XCD's L2 (the agent-scope
// load's sc1 bit, as the compiler emits for __hip_atomic_load at agent scope, here on a 16-byte
// load). The compiler does not track this load: the value may be used only after wait_loads().
__device__ __forceinline__ v4f load_coherent4(const float *p) {
    v4f r;
    asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(r) : "v"(p) : "memory");
    return r;
}
template <int N> __device__ __forceinline__ void wait_loads(v4f (&r)[N]) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" : "+v"(r[i])); // uses stay after the wait
}

// The merge of nslice chunk partials for each of ng query heads (attention.zig:113-133 merge):
// acc / ml point at the first head's sums [ng][nslice][HD] and {max, sum} pairs [ng][nslice][2],
// out at its output row [ng][HD]. The workgroup loads every (head, chunk) pair at once, one wave per
// head turns them into the weights exp(m_s - max m) of the non-empty chunks (in LDS: wts, lsh hold
// ng * nslice floats, tsh ng), and then each 16-byte output is summed over the chunks by tpo
// threads, sixteen chunks' loads at a time, all heads together. COH: the partials come from other
// workgroups of the same launch (loads at the coherence point).
template <bool COH, int HD>
__device__ void merge_chunks(const float *acc, const float *ml, float *out, uint32_t ng, uint32_t nslice, float *wts,
                             float *lsh, float *tsh, float *out_lds = nullptr) {
    auto ld = [&](const float *q) -> float {
        if constexpr (COH)
            return __hip_atomic_load(const_cast<float *>(q), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            return *q;
    };
    const uint32_t T = blockDim.x, lane = threadIdx.x & 63, NW = T >> 6, N = ng * nslice;
    for (uint32_t i0 = 0; i0 < N; i0 += 8 * T) {
        float m[8], l[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t i = i0 + threadIdx.x + k * T;
            if (i < N) {
                m[k] = ld(ml + ATT_ML * i);
                l[k] = ld(ml + ATT_ML * i + 1);
            }
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t i = i0 + threadIdx.x + k * T;
            if (i < N) {
                wts[i] = m[k];
                lsh[i] = l[k];
            }
        }
    }
    __syncthreads();
    for (uint32_t h = threadIdx.x >> 6; h < ng; h += NW) {
        float *w = wts + h * nslice;
        const float *l = lsh + h * nslice;
        float big = -INFINITY;
        for (uint32_t s = lane; s < nslice; s += 64)
            if (l[s] != 0.0f) big = fmaxf(big, w[s]);
        for (int o = 32; o >= 1; o >>= 1) big = fmaxf(big, __shfl_xor(big, o));
        float tot = 0.0f;
        for (uint32_t s = lane; s < nslice; s += 64) {
            const float wgt = l[s] != 0.0f ? expf(w[s] - big) : 0.0f;
            w[s] = wgt;
            tot = fmaf(wgt, l[s], tot);
        }
        for (int o = 32; o >= 1; o >>= 1) tot += __shfl_xor(tot, o);
        if (lane == 0) tsh[h] = tot;
    }
    __syncthreads();
    constexpr uint32_t Q = HD / 4;
    const uint32_t O = ng * Q;
    uint32_t tpo = 1; // threads per output: the largest power of two with tpo * O <= T
    while (2 * tpo * O <= T && tpo < 64) tpo *= 2;
    const uint32_t j = threadIdx.x % tpo;
    for (uint32_t o = threadIdx.x / tpo; o < O; o += T / tpo) {
        const uint32_t h = o / Q, d4 = o % Q;
        const float *base = acc + uint64_t(h) * nslice * HD + 4 * d4;
        const float *w = wts + h * nslice;
        v4f sum = v4f{};
        for (uint32_t s0 = j; s0 < nslice; s0 += 16 * tpo) {
            v4f r[16];
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const uint32_t sk = s0 + k * tpo;
                if (sk < nslice) {
                    if constexpr (COH)
                        r[k] = load_coherent4(base + uint64_t(sk) * HD);
                    else
                        r[k] = *reinterpret_cast<const v4f *>(base + uint64_t(sk) * HD);
                }
            }
            if constexpr (COH) wait_loads(r);
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const uint32_t sk = s0 + k * tpo;
                if (sk < nslice) sum += w[sk] * r[k];
            }
        }
        for (uint32_t m = 1; m < tpo; m <<= 1)
#pragma unroll
            for (int e = 0; e < 4; e++) sum[e] += __shfl_xor(sum[e], m);
        if (j == 0) {
            const v4f r = sum * (1.0f / tsh[h]);
            *reinterpret_cast<v4f *>(out + h * HD + 4 * d4) = r;
            if (out_lds) *reinterpret_cast<v4f *>(out_lds + h * HD + 4 * d4) = r; // the same values, for this workgroup
        }
    }
}

// Registers of a lane's share of the rope_dim / 2 rotation frequencies.
template <int HD> constexpr int rope_regs() { return (HD / 2 + 63) / 64; }
// cos and sin (times ropeMscale) of the lane's rotation angles pos * fr (ropeAngles, ops.zig:154-170).
template <int HD>
__device__ __forceinline__ void rope_cs(float (&cs)[rope_regs<HD>()], float (&sn)[rope_regs<HD>()],
                                        const float (&fr)[rope_regs<HD>()], uint32_t pos, const RopeArgs &a,
                                        uint32_t lane) {
    const float p = float(pos);
#pragma unroll
    for (int f = 0; f < rope_regs<HD>(); f++) {
        cs[f] = 0.0f;
        sn[f] = 0.0f;
        if (lane + 64 * f < a.rope_half) {
            float s_, c_;
            sincosf(p * fr[f], &s_, &c_);
            cs[f] = c_ * a.mscale;
            sn[f] = s_ * a.mscale;
        }
    }
}
// One row of HD values held by a wave (lane l: elements l + 64 j in x): headNorm (ops.zig:31-38,
// when nw_on) into the LDS row h, then the rotation of ropeApply (ops.zig:171-185) by the angles
// rope_cs gave, in place -- the steps head_norm_rope takes, from registers.
template <int HD>
__device__ __forceinline__ void norm_rope_row_cs(float *h, const float (&x)[HD / 64], const float (&nw)[HD / 64],
                                                 bool nw_on, const float (&cs)[rope_regs<HD>()],
                                                 const float (&sn)[rope_regs<HD>()], const RopeArgs &a, uint32_t lane) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < HD / 64; j++) ss = fmaf(x[j], x[j], ss);
    ss = wave_sum_f(ss);
    const float inv = nw_on ? __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, float(HD)) + a.eps)) : 1.0f;
#pragma unroll
    for (int j = 0; j < HD / 64; j++) h[lane + 64 * j] = nw_on ? (x[j] * inv) * nw[j] : x[j];
    wave_sync();
#pragma unroll
    for (int f = 0; f < rope_regs<HD>(); f++) {
        const uint32_t i = lane + 64 * f;
        if (i < a.rope_half) {
            const float c = cs[f], s = sn[f];
            const uint32_t i0 = a.neox ? i : 2 * i, i1 = a.neox ? i + a.rope_half : 2 * i + 1;
            const float x0 = h[i0], x1 = h[i1];
            h[i0] = x0 * c - x1 * s;
            h[i1] = x0 * s + x1 * c;
        }
    }
    wave_sync();
}
template <int HD>
__device__ __forceinline__ void norm_rope_row(float *h, const float (&x)[HD / 64], const float (&nw)[HD / 64], bool nw_on,
                                              const float (&fr)[rope_regs<HD>()], uint32_t pos, const RopeArgs &a,
                                              uint32_t lane) {
    float cs[rope_regs<HD>()], sn[rope_regs<HD>()];
    rope_cs<HD>(cs, sn, fr, pos, a, lane);
    norm_rope_row_cs<HD>(h, x, nw, nw_on, cs, sn, a, lane);
}

// The ng * HD results of token t's head block h0.. (the values this workgroup wrote to att, kept in
// its LDS row qo) quantized as whole Q8K blocks, one wave per block (qact_q8k_kernel's steps).
template <int HD, int NWV>
__device__ __forceinline__ void attn_quantize_block(const AttnArgs &a, uint32_t t, uint32_t h0, uint32_t ng,
                                                    const float *qo) {
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63, nb = ng * HD / QK_K, nsb = a.nh * HD / QK_K;
    for (uint32_t j = threadIdx.x >> 6; j < nb; j += NWV) {
        const float4 v = reinterpret_cast<const float4 *>(qo + QK_K * j)[lane];
        q8k_out(a.q8, uint64_t(t) * nsb + h0 * HD / QK_K + j, lane, quant_q8k_wave(v, lane));
    }
}

// The end of a decode attention workgroup, once its NWV waves' {max, sum, acc} of the ng (<= G)
// query heads h0.. are in red_m / red_l / red_acc (LDS, after a barrier): merges them per head and
// writes the normalized result (one chunk per (head, token)) or the chunk's partials, and the last
// chunk of (token, head block) to arrive merges every chunk's partials when a.cnt is set.
template <int HD, int NWV, int G>
__device__ __forceinline__ void attn_decode_finish(const AttnArgs &a, uint32_t g, uint32_t t, uint32_t h0, uint32_t ng,
                                                   const float (&red_m)[NWV][G], const float (&red_l)[NWV][G],
                                                   const float (&red_acc)[NWV][G][HD]) {
    // The waves' {max, sum, acc} per head (as the slice merge does, attention.zig:113-133).
    float big[G], tot[G], wt[G][NWV];
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        big[gi] = -INFINITY;
        const bool on = uint32_t(gi) < ng; // LDS of the heads past ng is not written
#pragma unroll
        for (int i = 0; i < NWV; i++)
            if (on && red_l[i][gi] != 0.0f) big[gi] = fmaxf(big[gi], red_m[i][gi]);
        tot[gi] = 0.0f;
#pragma unroll
        for (int i = 0; i < NWV; i++) {
            wt[gi][i] = on && red_l[i][gi] != 0.0f ? expf(red_m[i][gi] - big[gi]) : 0.0f;
            tot[gi] = fmaf(wt[gi][i], red_l[i][gi], tot[gi]);
        }
    }
    __shared__ float qo[G * HD]; // with q8_on: this workgroup's results, for attn_quantize_block
    if (a.att) { // one chunk: the normalized result (as attn_combine_kernel writes it)
#pragma unroll
        for (int gi = 0; gi < G; gi++) {
            if (uint32_t(gi) >= ng) break;
            const float inv = 1.0f / tot[gi];
            float *o = a.att + (uint64_t(t) * a.nh + h0 + gi) * HD;
            for (uint32_t d = threadIdx.x; d < HD; d += NWV * 64) {
                float v = 0.0f;
#pragma unroll
                for (int i = 0; i < NWV; i++) v = fmaf(wt[gi][i], red_acc[i][gi][d], v);
                o[d] = v * inv;
                if (a.q8_on) qo[gi * HD + d] = v * inv;
            }
        }
        if (a.q8_on) attn_quantize_block<HD, NWV>(a, t, h0, ng, qo);
        return;
    }
    // The chunk's partials per head: acc (unnormalized) and {max, sum}, as attn_combine_kernel reads
    // them. With the merge in this launch, they go out by agent-scope stores (they complete at the
    // device's coherent level, not in this XCD's L2).
    auto put = [&](float *out, uint32_t i, float v) {
        if (a.cnt)
            __hip_atomic_store(out + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            out[i] = v;
    };
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        if (uint32_t(gi) >= ng) break;
        const uint64_t pi = (uint64_t(t) * a.nh + h0 + gi) * gridDim.x + g;
        float *out = a.part + pi * HD;
        for (uint32_t d = threadIdx.x; d < HD; d += NWV * 64) {
            float v = 0.0f;
#pragma unroll
            for (int i = 0; i < NWV; i++) v = fmaf(wt[gi][i], red_acc[i][gi][d], v);
            put(out, d, v);
        }
        if (threadIdx.x == 0) {
            put(a.part_ml + ATT_ML * pi, 0, big[gi]);
            put(a.part_ml + ATT_ML * pi, 1, tot[gi]);
        }
    }
    if (!a.cnt) return; // attn_combine_kernel merges
    // Count the chunk in; the last of (token, head block) to arrive merges every chunk's partials.
    // No workgroup waits for another. Ordering: every access to the partials and the counter is an
    // agent-scope atomic, which gfx950 performs at the device's coherence point (stores written
    // through this XCD's L2, loads served past it), so a partial store is visible to every
    // workgroup once it has completed. Each wave therefore waits for its stores to complete
    // (vmcnt(0), with a compiler barrier) before the workgroup barrier, and only then does one
    // thread count the chunk in; the merging workgroup reads the partials only after it has seen
    // the final count. This is the code an agent-scope release / acquire pair generates on gfx950
    // minus its L2 write-back (buffer_wbl2) and invalidate (buffer_inv), which exist for
    // non-atomic data and which measured 7.5 us per Llama-3-8B layer at 512-575 positions (1.879
    // vs 1.637 ms per token; Qwen3-0.6B 0.949 vs 0.847).
    __shared__ uint32_t last;
    __shared__ float mw[G * ATT_MERGE_MAX], ml_[G * ATT_MERGE_MAX], mt[G];
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t *c = a.cnt + (uint64_t(t) * a.nh + h0) * ATT_CNT;
        last = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 == gridDim.x ? 1u : 0u;
        if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    const uint64_t p0 = (uint64_t(t) * a.nh + h0) * gridDim.x; // the block's first partial
    if (gridDim.x <= 8 && ng * HD <= 2 * NWV * 64) {
        // One round of loads per output: thread (head, d) reads every chunk's {max, sum, acc[d]} at once.
        for (uint32_t o = threadIdx.x; o < ng * HD; o += NWV * 64) {
            const uint32_t gi = o / HD, d = o % HD;
            float mm[8], ll[8], vv8[8];
#pragma unroll
            for (uint32_t i = 0; i < 8; i++) {
                if (i < gridDim.x) {
                    const uint64_t pi = p0 + gi * gridDim.x + i;
                    mm[i] = __hip_atomic_load(a.part_ml + ATT_ML * pi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ll[i] = __hip_atomic_load(a.part_ml + ATT_ML * pi + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    vv8[i] = __hip_atomic_load(a.part + pi * HD + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            float mx = -INFINITY;
#pragma unroll
            for (uint32_t i = 0; i < 8; i++)
                if (i < gridDim.x && ll[i] != 0.0f) mx = fmaxf(mx, mm[i]);
            float sum = 0.0f, av = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < 8; i++) {
                if (i < gridDim.x) {
                    const float wgt = ll[i] != 0.0f ? expf(mm[i] - mx) : 0.0f;
                    sum = fmaf(wgt, ll[i], sum);
                    av = fmaf(wgt, vv8[i], av);
                }
            }
            a.merge_out[(uint64_t(t) * a.nh + h0 + gi) * HD + d] = av * (1.0f / sum);
            if (a.q8_on) qo[gi * HD + d] = av * (1.0f / sum);
        }
    } else {
        merge_chunks<true, HD>(a.part + p0 * HD, a.part_ml + ATT_ML * p0, a.merge_out + (uint64_t(t) * a.nh + h0) * HD, ng,
                               gridDim.x, mw, ml_, mt, a.q8_on ? qo : nullptr);
    }
    if (a.q8_on) attn_quantize_block<HD, NWV>(a, t, h0, ng, qo);
}

// G query heads h0 .. h0 + G - 1 that share one key/value head (G divides the group size: the
// whole group, or 1) per workgroup, so each key and value row is loaded once for all of them.
template <int HD, int NWV, int G>
__global__ __launch_bounds__(NWV * 64) void attn_decode_kernel(AttnArgs a) {
    constexpr int LPR = HD / 8, RPI = 64 / LPR, NI = 64 / RPI; // lanes per value row, rows per load, loads
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t vr_ = lane / LPR, vc = lane % LPR; // value row within a load, dimension chunk
    const uint32_t g = blockIdx.x, t = blockIdx.z;
    const uint32_t grp = a.nh / a.nkv, h0 = blockIdx.y * G, kvh = h0 / grp;
    __shared__ float qs[G][HD];
    __shared__ float red_m[NWV][G], red_l[NWV][G];
    __shared__ float prs[NWV][G][64]; // a step's probabilities per head, for the value rows' lanes
    __shared__ float red_acc[NWV][G][HD];
    __shared__ float kn[HD];                                  // fused: the new key row, f32
    __shared__ __attribute__((aligned(16))) __half kvh16[2][HD]; // fused: new key / value rows, f16
    const uint64_t sl = a.slot[t];
    const uint32_t pos = a.pos[t];
    const __half *kb = a.kc + sl * a.kv_slot + uint64_t(kvh) * a.max_ctx * HD;
    const __half *vb = a.vc + sl * a.kv_slot + uint64_t(kvh) * a.max_ctx * HD + 8 * vc;
    // The q rows of this wave's heads (w, w + NWV, ... of the G), and for a one-token (fused) pass
    // the norm weights, the rotation frequencies and the raw new key / value rows, are loaded before
    // the cache rows: the memory counter is in order, so the q rows' norm and rotation then run
    // while the cache rows are in flight.
    constexpr int QPW = (G + NWV - 1) / NWV;
    float qv[QPW][HD / 64], qnw[HD / 64], kx[HD / 64], knw[HD / 64], vx[HD / 64], fr[rope_regs<HD>()];
#pragma unroll
    for (int qi = 0; qi < QPW; qi++) {
        const uint32_t gi = w + NWV * qi;
        const float *qsrc = a.q + uint64_t(t) * a.sq + (h0 + (gi < uint32_t(G) ? gi : 0)) * HD;
#pragma unroll
        for (int j = 0; j < HD / 64; j++) qv[qi][j] = qsrc[lane + 64 * j];
    }
    if (a.fused) {
#pragma unroll
        for (int j = 0; j < HD / 64; j++) {
            qnw[j] = a.r.q_norm ? a.r.q_norm[lane + 64 * j] : 1.0f;
            knw[j] = a.r.k_norm ? a.r.k_norm[lane + 64 * j] : 1.0f;
            kx[j] = a.r.k[uint64_t(t) * a.r.skv + kvh * HD + lane + 64 * j];
            vx[j] = a.r.v[uint64_t(t) * a.r.skv + kvh * HD + lane + 64 * j];
        }
#pragma unroll
        for (int f = 0; f < rope_regs<HD>(); f++) fr[f] = lane + 64 * f < a.r.rope_half ? a.r.inv_freq[lane + 64 * f] : 0.0f;
    }
    // The launch gives every 64-position step of the context a wave of its own, so a wave has one
    // step, and its loads need not wait for the position: rows are clamped to the cache only, and
    // rows past the token's position (finite: the caches start zeroed) are masked.
    const uint32_t p0 = 64 * (g * NWV + w);
    const uint32_t pp = p0 + lane, lastc = a.max_ctx - 1;
    uint4 kr[HD / 8], vv[NI];
    {
        const uint4 *krow = reinterpret_cast<const uint4 *>(kb + uint64_t(pp < lastc ? pp : lastc) * HD);
#pragma unroll
        for (int c = 0; c < HD / 8; c++) kr[c] = krow[c];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const uint32_t pv = p0 + RPI * i + vr_;
            vv[i] = *reinterpret_cast<const uint4 *>(vb + uint64_t(pv < lastc ? pv : lastc) * HD);
        }
    }
    // The q rows to LDS; a one-token pass normalizes and rotates them (rope_kv_kernel's steps,
    // which the multi-token passes ran before this kernel).
#pragma unroll
    for (int qi = 0; qi < QPW; qi++) {
        const uint32_t gi = w + NWV * qi;
        if (gi < uint32_t(G)) {
            if (a.fused) {
                norm_rope_row<HD>(qs[gi], qv[qi], qnw, a.r.q_norm != nullptr, fr, pos, a.r, lane);
            } else {
#pragma unroll
                for (int j = 0; j < HD / 64; j++) qs[gi][lane + 64 * j] = qv[qi][j];
            }
        }
    }
    __syncthreads();
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        m[gi] = -INFINITY;
        l[gi] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) acc[gi][j] = 0.0f;
    }
    if (p0 <= pos) {
        const uint32_t p_end = min(p0 + 64, pos + 1);
        // Fused pass, wave holding the new position: its scores (in the order of the cache rows'
        // dots below) and value row (vnew) replace what the loads brought for that position.
        const bool has_new = a.fused && pos < p0 + 64;
        float dot_new[G];
        uint4 vnew = make_uint4(0, 0, 0, 0);
        if (has_new) {
            norm_rope_row<HD>(kn, kx, knw, a.r.k_norm != nullptr, fr, pos, a.r, lane);
#pragma unroll
            for (int j = 0; j < HD / 64; j++) {
                kvh16[0][lane + 64 * j] = __float2half(kn[lane + 64 * j]);
                kvh16[1][lane + 64 * j] = __float2half(vx[j]);
            }
            wave_sync();
#pragma unroll
            for (int gi = 0; gi < G; gi++) {
                float dn = 0.0f;
                for (int c = 0; c < HD / 8; c++) {
                    const uint4 kw = reinterpret_cast<const uint4 *>(kvh16[0])[c];
                    const __half2 *hp = reinterpret_cast<const __half2 *>(&kw);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float2 f = __half22float2(hp[e]);
                        dn = fmaf(qs[gi][8 * c + 2 * e], f.x, dn);
                        dn = fmaf(qs[gi][8 * c + 2 * e + 1], f.y, dn);
                    }
                }
                dot_new[gi] = dn;
            }
            vnew = *reinterpret_cast<const uint4 *>(&kvh16[1][8 * vc]);
            if (h0 % grp == 0) { // one writer per key/value head
                __half *kd = a.r.kc + sl * a.r.kv_slot + (uint64_t(kvh) * a.max_ctx + pos) * HD;
                __half *vd = a.r.vc + sl * a.r.kv_slot + (uint64_t(kvh) * a.max_ctx + pos) * HD;
                __half *vtd = a.r.vt + sl * a.r.vt_slot + uint64_t(kvh) * HD * a.r.vt_stride + pos;
#pragma unroll
                for (int j = 0; j < HD / 64; j++) {
                    const uint32_t d = lane + 64 * j;
                    kd[d] = kvh16[0][d];
                    vd[d] = kvh16[1][d];
                    vtd[uint64_t(d) * a.r.vt_stride] = kvh16[1][d];
                }
            }
        }
#pragma unroll
        for (int c = 0; c < HD / 8; c++) asm volatile("" : "+v"(kr[c].x), "+v"(kr[c].y), "+v"(kr[c].z), "+v"(kr[c].w));
#pragma unroll
        for (int i = 0; i < NI; i++) asm volatile("" : "+v"(vv[i].x), "+v"(vv[i].y), "+v"(vv[i].z), "+v"(vv[i].w));
        float dot[G];
#pragma unroll
        for (int gi = 0; gi < G; gi++) dot[gi] = 0.0f;
#pragma unroll
        for (int c = 0; c < HD / 8; c++) {
            const __half2 *hp = reinterpret_cast<const __half2 *>(&kr[c]);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float2 f = __half22float2(hp[e]);
#pragma unroll
                for (int gi = 0; gi < G; gi++) {
                    dot[gi] = fmaf(qs[gi][8 * c + 2 * e], f.x, dot[gi]);
                    dot[gi] = fmaf(qs[gi][8 * c + 2 * e + 1], f.y, dot[gi]);
                }
            }
        }
        float corr[G];
#pragma unroll
        for (int gi = 0; gi < G; gi++) {
            if (has_new && pp == pos) dot[gi] = dot_new[gi];
            const float s = pp < p_end ? dot[gi] * a.scale : -INFINITY;
            const float mn = fmaxf(m[gi], wave_max_f(s));
            const float pr = pp < p_end ? expf(s - mn) : 0.0f;
            const float ps = wave_sum_f(pr);
            prs[w][gi][lane] = pr;
            corr[gi] = m[gi] == -INFINITY ? 0.0f : expf(m[gi] - mn);
            l[gi] = l[gi] * corr[gi] + ps;
            m[gi] = mn;
        }
        wave_sync();
#pragma unroll
        for (int gi = 0; gi < G; gi++)
#pragma unroll
            for (int j = 0; j < 8; j++) acc[gi][j] *= corr[gi];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const uint4 vw = has_new && p0 + RPI * i + vr_ == pos ? vnew : vv[i];
            const __half2 *hp = reinterpret_cast<const __half2 *>(&vw);
            float vf[8];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float2 f = __half22float2(hp[e]);
                vf[2 * e] = f.x;
                vf[2 * e + 1] = f.y;
            }
#pragma unroll
            for (int gi = 0; gi < G; gi++) {
                const float pi = prs[w][gi][RPI * i + vr_]; // 0 for positions past the step
#pragma unroll
                for (int e = 0; e < 8; e++) acc[gi][e] = fmaf(pi, vf[e], acc[gi][e]);
            }
        }
    }
    // The RPI row groups' sums of each dimension chunk (lanes vc, vc + LPR, ...).
#pragma unroll
    for (int o = LPR; o < 64; o <<= 1)
#pragma unroll
        for (int gi = 0; gi < G; gi++)
#pragma unroll
            for (int j = 0; j < 8; j++) acc[gi][j] += __shfl_xor(acc[gi][j], o);
    if (lane == 0) {
#pragma unroll
        for (int gi = 0; gi < G; gi++) {
            red_m[w][gi] = m[gi];
            red_l[w][gi] = l[gi];
        }
    }
    if (lane < LPR) {
#pragma unroll
        for (int gi = 0; gi < G; gi++)
#pragma unroll
            for (int j = 0; j < 8; j++) red_acc[w][gi][8 * lane + j] = acc[gi][j];
    }
    __syncthreads();
    attn_decode_finish<HD, NWV, G>(a, g, t, h0, G, red_m, red_l, red_acc);
}


// Decode attention of non-fused passes on the f16 MFMA units (v_mfma_f32_16x16x32_f16), one
// workgroup per (chunk, block of ng <= 8 query heads sharing one key/value head, token): the key
// and value rows of a position are loaded once for the whole block. Chunks, waves and the result
// (partials, the in-launch merge) are as in attn_decode_kernel; wave w of chunk g takes the PB
// blocks of 32 positions from p0 = 32 PB (g NWV + w), and being the only step of its wave, needs no
// running rescale. Per block of 32 positions:
//   S^T[pos][col] = K[pos] . Q[col]: A = key rows (f16, exact), B = the block's q rows split as
//       f16 hi (columns 0..7, head = column) and lo = q - hi (columns 8..15), so that a score is
//       column c's plus column c ^ 8's (q to ~2^-22, as attn_prefill_kernel does in two chains);
//   O^T[dim][col] += V^T[dim][pos] . P[pos][col]: A = the transposed value cache, B = the
//       probabilities split as f16 hi (columns 0..7) and lo (8..15).
// The block's two score tiles take its key rows in the order that leaves lane (column c, group q)
// holding positions 8q .. 8q + 7 of the block, exactly the k slots of the second product's B
// operand, so the probabilities feed it without moving.
template <int HD, int NWV, int PB, bool FUSED>
__global__ __launch_bounds__(NWV * 64) void attn_decode_gqa_kernel(AttnArgs a, uint32_t ng) {
    constexpr int NS = HD / 32, NDT = HD / 16; // k steps of the scores, dimension tiles of the output
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t c = lane & 15, qg = lane >> 4, hq = c & 7;
    const uint32_t g = blockIdx.x, t = blockIdx.z;
    const uint32_t grp = a.nh / a.nkv, h0 = blockIdx.y * ng, kvh = h0 / grp;
    __shared__ float red_m[NWV][8], red_l[NWV][8];
    __shared__ float red_acc[NWV][8][HD];
    const uint64_t sl = a.slot[t];
    const uint32_t pos = a.pos[t];
    // q operands first (the memory counter is in order): lane (c, q) holds dimensions
    // 32 s + 8 q .. + 8 of head hq's hi (c < 8) or lo part, zero for columns past the block.
    // Fused (every token of the pass in its own slot): the raw q rows of this wave's heads, the norm
    // weights, the inverse frequencies and the token's raw new key and value rows instead, ahead of
    // the cache rows; the operands are built from the normalized, rotated rows below.
    v8h qb[NS];
    float4 xq[NS][2];                                                          // fused: raw q
    float qnw[HD / 64], knw[HD / 64], kx[HD / 64], vx[HD / 64], fr[rope_regs<HD>()]; // norms, new key / value
    if constexpr (FUSED) {
        const float *qrow = a.q + uint64_t(t) * a.sq + (h0 + (hq < ng ? hq : 0)) * HD + 8 * qg;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            xq[s][0] = *reinterpret_cast<const float4 *>(qrow + 32 * s);
            xq[s][1] = *reinterpret_cast<const float4 *>(qrow + 32 * s + 4);
        }
        const float *ksrc = a.r.k + uint64_t(t) * a.r.skv + kvh * HD, *vsrc = a.r.v + uint64_t(t) * a.r.skv + kvh * HD;
#pragma unroll
        for (int j = 0; j < HD / 64; j++) {
            qnw[j] = a.r.q_norm ? a.r.q_norm[lane + 64 * j] : 1.0f;
            knw[j] = a.r.k_norm ? a.r.k_norm[lane + 64 * j] : 1.0f;
            kx[j] = ksrc[lane + 64 * j];
            vx[j] = vsrc[lane + 64 * j];
        }
#pragma unroll
        for (int f = 0; f < rope_regs<HD>(); f++) fr[f] = lane + 64 * f < a.r.rope_half ? a.r.inv_freq[lane + 64 * f] : 0.0f;
    } else {
        const float *qrow = a.q + uint64_t(t) * a.sq + (h0 + (hq < ng ? hq : 0)) * HD + 8 * qg;
        float4 x[NS][2];
#pragma unroll
        for (int s = 0; s < NS; s++) {
            x[s][0] = *reinterpret_cast<const float4 *>(qrow + 32 * s);
            x[s][1] = *reinterpret_cast<const float4 *>(qrow + 32 * s + 4);
        }
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const float xs[8] = {x[s][0].x, x[s][0].y, x[s][0].z, x[s][0].w, x[s][1].x, x[s][1].y, x[s][1].z, x[s][1].w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const _Float16 hi = (_Float16)xs[e];
                const _Float16 v = c < 8 ? hi : (_Float16)(xs[e] - (float)hi);
                qb[s][e] = hq < ng ? v : (_Float16)0.0f;
            }
        }
    }
    const uint32_t p0 = 32 * PB * (g * NWV + w), lastc = a.max_ctx - 1;
    // Key rows: tile (b, u) row c is position 32 b + 8 (c / 4) + 4 u + c % 4; value rows: dimension
    // 16 d + c, positions 32 b + 8 q .. + 8. Clamped to the caches only (rows past the token's
    // position are masked; the caches start zeroed, so they are finite).
    v8h ka[PB][2][NS], va[PB][NDT];
    {
        const __half *kb = a.kc + sl * a.kv_slot + uint64_t(kvh) * a.max_ctx * HD + 8 * qg;
        const __half *vb = a.r.vt + sl * a.r.vt_slot + uint64_t(kvh) * HD * a.r.vt_stride + 8 * qg;
#pragma unroll
        for (int b = 0; b < PB; b++) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const uint32_t kp = p0 + 32 * b + 8 * (c >> 2) + 4 * u + (c & 3);
                const __half *krow = kb + uint64_t(kp < lastc ? kp : lastc) * HD;
#pragma unroll
                for (int s = 0; s < NS; s++) ka[b][u][s] = *reinterpret_cast<const v8h *>(krow + 32 * s);
            }
            const uint32_t vp = min(p0 + 32 * b, a.r.vt_stride - 32);
#pragma unroll
            for (int d = 0; d < NDT; d++)
                va[b][d] = *reinterpret_cast<const v8h *>(vb + uint64_t(16 * d + c) * a.r.vt_stride + vp);
        }
    }
    // Every row in flight before the first use (the compiler would otherwise sink each load next
    // to its product).
#pragma unroll
    for (int b = 0; b < PB; b++) {
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int s = 0; s < NS; s++) asm volatile("" : "+v"(ka[b][u][s]));
#pragma unroll
        for (int d = 0; d < NDT; d++) asm volatile("" : "+v"(va[b][d]));
    }
    if constexpr (FUSED) {
        // q in the operand layout, in registers: a head's sum of squares is its lanes' partials over
        // the four lane groups (headNorm, ops.zig:31-38), and every rotation pair (ropeApply,
        // ops.zig:171-185) lies in one lane -- (i, i + rope_half) two or one k steps apart (neox,
        // rope_half a multiple of 32: the host's condition), (2i, 2i + 1) neighbours (pairwise) --
        // with the angles' cos / sin from a table each wave writes (identical values) to LDS. In the
        // chunk holding the token's position one wave builds the new key row as rope_kv_kernel
        // does, and both new rows go to f16.
        __shared__ float cst[2][HD / 2], qwt[HD], knf[HD];
        __shared__ __attribute__((aligned(16))) _Float16 kv16[2][HD];
        float cs[rope_regs<HD>()], sn[rope_regs<HD>()];
        rope_cs<HD>(cs, sn, fr, pos, a.r, lane);
#pragma unroll
        for (int j = 0; j < HD / 64; j++) qwt[lane + 64 * j] = qnw[j]; // identical in every wave
#pragma unroll
        for (int f = 0; f < rope_regs<HD>(); f++)
            if (lane + 64 * f < a.r.rope_half) {
                cst[0][lane + 64 * f] = cs[f];
                cst[1][lane + 64 * f] = sn[f];
            }
        float y[NS][8];
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const float v[8] = {xq[s][0].x, xq[s][0].y, xq[s][0].z, xq[s][0].w, xq[s][1].x, xq[s][1].y, xq[s][1].z, xq[s][1].w};
#pragma unroll
            for (int e = 0; e < 8; e++) y[s][e] = v[e];
        }
        wave_sync(); // the norm weights and the angle table
        if (a.r.q_norm) {
            float ss = 0.0f;
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int e = 0; e < 8; e++) ss = fmaf(y[s][e], y[s][e], ss);
            ss += __shfl_xor(ss, 16);
            ss += __shfl_xor(ss, 32);
            const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, float(HD)) + a.r.eps));
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int e = 0; e < 8; e++) y[s][e] = (y[s][e] * inv) * qwt[32 * s + 8 * qg + e];
        }
        const uint32_t rh = a.r.rope_half;
        if (a.r.neox) {
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int s2 = s + 1; s2 < NS; s2++)
                    if (uint32_t(32 * (s2 - s)) == rh && uint32_t(32 * s) < rh)
#pragma unroll
                        for (int e = 0; e < 8; e++) {
                            const uint32_t i = 32 * s + 8 * qg + e;
                            const float cc = cst[0][i], sc = cst[1][i], x0 = y[s][e], x1 = y[s2][e];
                            y[s][e] = x0 * cc - x1 * sc;
                            y[s2][e] = x0 * sc + x1 * cc;
                        }
        } else {
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const uint32_t i = (32 * s + 8 * qg + e) / 2;
                    if (i < rh) {
                        const float cc = cst[0][i], sc = cst[1][i], x0 = y[s][e], x1 = y[s][e + 1];
                        y[s][e] = x0 * cc - x1 * sc;
                        y[s][e + 1] = x0 * sc + x1 * cc;
                    }
                }
        }
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float xv = hq < ng ? y[s][e] : 0.0f;
                const _Float16 hi = (_Float16)xv;
                qb[s][e] = c < 8 ? hi : (_Float16)(xv - (float)hi);
            }
        const bool own = pos / (32 * PB * NWV) == g; // uniform over the workgroup
        if (own) {
            if (w == NWV - 1) {
                norm_rope_row_cs<HD>(knf, kx, knw, a.r.k_norm != nullptr, cs, sn, a.r, lane);
#pragma unroll
                for (int j = 0; j < HD / 64; j++) {
                    kv16[0][lane + 64 * j] = (_Float16)knf[lane + 64 * j];
                    kv16[1][lane + 64 * j] = (_Float16)vx[j];
                }
            }
            __syncthreads();
        }
        if (own) {
            // The loads brought the cache's old rows for the token's position: the new ones replace
            // them, and the first head block of the key/value head writes them to the caches (no
            // other workgroup of the launch reads this position of this slot).
#pragma unroll
            for (int b = 0; b < PB; b++) {
#pragma unroll
                for (int u = 0; u < 2; u++)
                    if (p0 + 32 * b + 8 * (c >> 2) + 4 * u + (c & 3) == pos)
#pragma unroll
                        for (int s = 0; s < NS; s++) ka[b][u][s] = *reinterpret_cast<const v8h *>(&kv16[0][32 * s + 8 * qg]);
                const uint32_t base = p0 + 32 * b + 8 * qg;
                if (pos >= base && pos < base + 8) {
#pragma unroll
                    for (int d = 0; d < NDT; d++) {
                        const _Float16 nv = kv16[1][16 * d + c];
#pragma unroll
                        for (int e = 0; e < 8; e++)
                            if (base + e == pos) va[b][d][e] = nv;
                    }
                }
            }
            if (h0 % grp == 0) {
                const __half *k16 = reinterpret_cast<const __half *>(kv16[0]), *v16 = reinterpret_cast<const __half *>(kv16[1]);
                __half *kd = a.r.kc + sl * a.r.kv_slot + (uint64_t(kvh) * a.max_ctx + pos) * HD;
                __half *vd = a.r.vc + sl * a.r.kv_slot + (uint64_t(kvh) * a.max_ctx + pos) * HD;
                __half *vtd = a.r.vt + sl * a.r.vt_slot + uint64_t(kvh) * HD * a.r.vt_stride + pos;
                for (uint32_t d = threadIdx.x; d < HD; d += NWV * 64) {
                    kd[d] = k16[d];
                    vd[d] = v16[d];
                    vtd[uint64_t(d) * a.r.vt_stride] = v16[d];
                }
            }
        }
    }
    float mx = -INFINITY, lsum = 0.0f;
    v4f o[NDT];
#pragma unroll
    for (int d = 0; d < NDT; d++) o[d] = v4f{};
    if (p0 <= pos) {
        float sv[PB][8];
#pragma unroll
        for (int b = 0; b < PB; b++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                v4f sc = v4f{};
#pragma unroll
                for (int s = 0; s < NS; s++) sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[b][u][s], qb[s], sc, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float v = sc[i] + dpp_f<DPP_ROR8>(sc[i]); // hi + lo columns
                    const uint32_t pp = p0 + 32 * b + 8 * qg + 4 * u + i;
                    sv[b][4 * u + i] = pp <= pos ? v * a.scale : -INFINITY;
                    mx = fmaxf(mx, sv[b][4 * u + i]);
                }
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32)); // finite: position p0 is unmasked
        v8h pb[PB];
#pragma unroll
        for (int b = 0; b < PB; b++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float p = expf(sv[b][e] - mx); // 0 where masked
                lsum += p;
                const _Float16 hi = (_Float16)p;
                pb[b][e] = c < 8 ? hi : (_Float16)(p - (float)hi);
            }
        lsum += __shfl_xor(lsum, 16);
        lsum += __shfl_xor(lsum, 32);
#pragma unroll
        for (int b = 0; b < PB; b++)
#pragma unroll
            for (int d = 0; d < NDT; d++) o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[b][d], pb[b], o[d], 0, 0, 0);
    }
    // Lane (c, q) holds dimensions 16 d + 4 q + i of column c: a head's sums are columns c and c ^ 8.
#pragma unroll
    for (int d = 0; d < NDT; d++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float v = o[d][i] + dpp_f<DPP_ROR8>(o[d][i]);
            if (c < ng) red_acc[w][c][16 * d + 4 * qg + i] = v;
        }
    }
    if (qg == 0 && c < ng) {
        red_m[w][c] = mx;
        red_l[w][c] = lsum;
    }
    __syncthreads();
    attn_decode_finish<HD, NWV, 8>(a, g, t, h0, ng, red_m, red_l, red_acc);
}

// Prefill attention (passes of more than MAX_DECODE tokens) on the f16 MFMA units, one workgroup
// per (32-token tile, query head), the tiles with the most positions first; its NWV waves take
// every NWV-th tile of 32 positions and merge their partial results through LDS at the end (max /
// sum rescaling, as the slice merge does).
// Per tile of 32 positions:
//   S^T[pos][tok] = K[pos] . q[tok]: A = key rows (f16, exact), B = q split as f16 hi + lo (q - hi
//       rounded again; together q to ~2^-22), two MFMA chains over head_dim in steps of 16;
//   online softmax per token (a lane holds one token's 16 scores; the two lane halves meet by one
//       exchange), the scores scaled and masked as attn_slice_kernel does;
//   O^T[dim][tok] += V^T[dim][pos] . P^T[pos][tok]: A = the transposed value cache (positions
//       contiguous per dimension), B = the probabilities split as f16 hi + lo.
// The key rows are loaded in the order rho (bits 2 and 3 of the row swapped), which puts each
// lane half's 16 scores exactly on the 8 + 8 positions the second product's B operand needs, so
// the probabilities go from the first product's output to the second's input without moving.
struct AttnPArgs {
    const float *q;
    const __half *kc, *vt; // this layer's key cache [nkv][max_ctx][hd], value cache transposed [nkv][hd][vt_stride], slot 0
    float *att;
    const uint32_t *pos, *slot; // of the run's first token: the run is positions pos[0].. of slot slot[0]
    uint64_t kv_slot, vt_slot;
    uint32_t n, nh, nkv, max_ctx, vt_stride;
    float scale;
    uint32_t sq; // q row stride (floats per token)
};

// LDS of attn_prefill_kernel<HD, NWV>: the q operands, then the merge area of waves 1..NWV-1.
template <int HD, int NWV> struct AttnPSmem {
    v8h qsh[HD / 16][64], qsl[HD / 16][64];
    float red_m[NWV - 1][64], red_l[NWV - 1][64];
    float4 red_acc[NWV - 1][HD / 8][64];
};

template <int HD, int NWV>
__global__ __launch_bounds__(NWV * 64, 2) void attn_prefill_kernel(AttnPArgs a) {
    constexpr int NCH = HD / 16, NDT = HD / 32;
    extern __shared__ __attribute__((aligned(16))) uint8_t attn_smem[];
    AttnPSmem<HD, NWV> &S = *reinterpret_cast<AttnPSmem<HD, NWV> *>(attn_smem);
    const uint32_t lane = threadIdx.x & 63, h = lane >> 5, j = lane & 31;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t item = blockIdx.x; // < ntile * nh (the grid)
    const uint32_t ntile = (a.n + 31) / 32;
    const uint32_t head = item % a.nh, tile = ntile - 1 - item / a.nh; // longest prefixes first
    const uint32_t kvh = head / (a.nh / a.nkv);
    const uint32_t pos0 = a.pos[0];
    const uint64_t sl = a.slot[0];
    const uint32_t t = tile * 32 + j, tc = t < a.n ? t : a.n - 1; // this lane's token (clamped)
    const uint32_t tpos = pos0 + tc;
    const uint32_t tfirst = pos0 + tile * 32; // the tile's first token position (lane 0's)
    const uint32_t pend = pos0 + min(tile * 32 + 32, a.n); // positions [0, pend) are needed

    // The tile's q operands (the same 32 tokens for the four waves) live in LDS, split over the
    // waves' lanes to build, so that they take no registers: with them in registers the kernel
    // held one workgroup per CU.
    auto &qsh = S.qsh;
    auto &qsl = S.qsl;
    {
        const float *qrow = a.q + uint64_t(tc) * a.sq + head * HD;
        for (int c = int(wave); c < NCH; c += NWV) {
            const float4 x0 = *reinterpret_cast<const float4 *>(qrow + 16 * c + 8 * h);
            const float4 x1 = *reinterpret_cast<const float4 *>(qrow + 16 * c + 8 * h + 4);
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            v8h hv, lv;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const _Float16 hi = (_Float16)xs[e];
                hv[e] = hi;
                lv[e] = (_Float16)(xs[e] - (float)hi);
            }
            qsh[c][lane] = hv;
            qsl[c][lane] = lv;
        }
    }
    __syncthreads();
    v16f acc[NDT];
#pragma unroll
    for (int d = 0; d < NDT; d++) acc[d] = v16f{};
    float m = -INFINITY, l = 0.0f;
    const __half *kb = a.kc + sl * a.kv_slot + uint64_t(kvh) * a.max_ctx * HD;
    const __half *vb = a.vt + sl * a.vt_slot + uint64_t(kvh) * HD * a.vt_stride;
    const uint32_t rj = (j & ~12u) | ((j & 4u) << 1) | ((j & 8u) >> 1); // rho(j)
    // The key rows of the next tile of positions are loaded once this tile's scores are issued,
    // and its value rows once this tile's output products are: each lands while the other half
    // of the step runs, with no second set of registers.
    v8h ka[NCH], va[NDT][2];
    auto load_k = [&](uint32_t p0) {
        const uint32_t kp = p0 + rj < a.max_ctx ? p0 + rj : a.max_ctx - 1;
        const v8h *krow = reinterpret_cast<const v8h *>(kb + uint64_t(kp) * HD);
#pragma unroll
        for (int c = 0; c < NCH; c++) ka[c] = krow[2 * c + h];
    };
    auto load_v = [&](uint32_t p0) {
#pragma unroll
        for (int d = 0; d < NDT; d++)
#pragma unroll
            for (int cc = 0; cc < 2; cc++)
                va[d][cc] = *reinterpret_cast<const v8h *>(vb + uint64_t(32 * d + j) * a.vt_stride + p0 + 16 * cc + 8 * h);
    };
    if (32 * wave < pend) {
        load_k(32 * wave);
        load_v(32 * wave);
    }
    for (uint32_t p0 = 32 * wave; p0 < pend; p0 += 32 * NWV) {
        const uint32_t pn = p0 + 32 * NWV;
        v16f s = v16f{};
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[c], qsh[c][lane], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[c], qsl[c][lane], s, 0, 0, 0);
        }
        if (pn < pend) load_k(pn);
        // Score v of this lane: position p0 + 16(g >> 1) + 8h + 4(g & 1) + e, g = v / 4, e = v % 4.
        // Only the tiles reaching past the tile's first token position are masked.
        float sv[16], mx = -INFINITY;
        if (p0 + 31 > tfirst) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int g = v / 4, e = v % 4;
                const uint32_t pp = p0 + 16 * (g >> 1) + 8 * h + 4 * (g & 1) + e;
                sv[v] = pp <= tpos ? s[v] * a.scale : -INFINITY;
                mx = fmaxf(mx, sv[v]);
            }
        } else {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                sv[v] = s[v] * a.scale;
                mx = fmaxf(mx, sv[v]);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        // The hardware exponential (v_exp_f32 on x * log2 e: relative error ~1e-6 over the
        // softmax's range x <= 0), measured 1 us of the 17 us of a 512-token Llama-3-8B layer.
        const float corr = m == -INFINITY ? 0.0f : __expf(m - mn);
        float pv[16], ps = 0.0f;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            pv[v] = sv[v] == -INFINITY ? 0.0f : __expf(sv[v] - mn);
            ps += pv[v];
        }
        ps += __shfl_xor(ps, 32);
        l = l * corr + ps;
        m = mn;
        // The running sums need rescaling only where some lane's maximum moved.
        if (__any(corr != 1.0f)) {
#pragma unroll
            for (int d = 0; d < NDT; d++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[d][v] *= corr;
        }
#pragma unroll
        for (int cc = 0; cc < 2; cc++) {
            v8h ph, pl;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const _Float16 hi = (_Float16)pv[8 * cc + e];
                ph[e] = hi;
                pl[e] = (_Float16)(pv[8 * cc + e] - (float)hi);
            }
#pragma unroll
            for (int d = 0; d < NDT; d++) {
                acc[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[d][cc], ph, acc[d], 0, 0, 0);
                acc[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[d][cc], pl, acc[d], 0, 0, 0);
            }
        }
        if (pn < pend) load_v(pn);
    }
    // Merge: waves 1.. leave {m, l, acc} in LDS (a wave without tiles: m = -inf, l = 0), wave 0
    // rescales all of them to the common maximum, sums and writes.
    auto &red_m = S.red_m;
    auto &red_l = S.red_l;
    auto &red_acc = S.red_acc;
    if (wave > 0) {
        red_m[wave - 1][lane] = m;
        red_l[wave - 1][lane] = l;
#pragma unroll
        for (int d = 0; d < NDT; d++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                red_acc[wave - 1][4 * d + g][lane] = make_float4(acc[d][4 * g], acc[d][4 * g + 1], acc[d][4 * g + 2], acc[d][4 * g + 3]);
    }
    __syncthreads();
    if (wave > 0) return;
    float big = m;
#pragma unroll
    for (int w = 0; w < NWV - 1; w++) big = fmaxf(big, red_m[w][lane]);
    const float c0 = m == -INFINITY ? 0.0f : expf(m - big);
    float lt = l * c0, cw[NWV - 1];
#pragma unroll
    for (int w = 0; w < NWV - 1; w++) {
        const float mw = red_m[w][lane];
        cw[w] = mw == -INFINITY ? 0.0f : expf(mw - big);
        lt = fmaf(red_l[w][lane], cw[w], lt);
    }
    if (t < a.n) {
        // acc[d][v]: dimension 32d + 8g + 4h + e of this lane's token.
        const float inv = 1.0f / lt;
        float *o = a.att + (uint64_t(t) * a.nh + head) * HD;
#pragma unroll
        for (int d = 0; d < NDT; d++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                float4 r = make_float4(acc[d][4 * g] * c0, acc[d][4 * g + 1] * c0, acc[d][4 * g + 2] * c0, acc[d][4 * g + 3] * c0);
#pragma unroll
                for (int w = 0; w < NWV - 1; w++) {
                    const float4 x = red_acc[w][4 * d + g][lane];
                    r.x = fmaf(x.x, cw[w], r.x);
                    r.y = fmaf(x.y, cw[w], r.y);
                    r.z = fmaf(x.z, cw[w], r.z);
                    r.w = fmaf(x.w, cw[w], r.w);
                }
                *reinterpret_cast<float4 *>(o + 32 * d + 8 * g + 4 * h) = make_float4(r.x * inv, r.y * inv, r.z * inv, r.w * inv);
            }
    }
}

template <int HD, int NWV> hipError_t launch_attn_prefill(dim3 grid, const AttnPArgs &pa, hipStream_t s) {
    constexpr size_t lds = sizeof(AttnPSmem<HD, NWV>);
    static_assert(lds <= 160 * 1024, "LDS");
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_prefill_kernel<HD, NWV>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        attr = true;
    }
    hipLaunchKernelGGL((attn_prefill_kernel<HD, NWV>), grid, dim3(NWV * 64), lds, s, pa);
    return hipGetLastError();
}

// att[t][h*hd..] = merge of the slices' partials of (head h, token t).
template <int HD>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float *__restrict__ part, const float *__restrict__ part_ml,
                                                           float *__restrict__ att, uint32_t nh, uint32_t nslice) {
    extern __shared__ float wts[]; // [2 * nslice]
    __shared__ float tot[1];
    const uint64_t th = uint64_t(blockIdx.y) * nh + blockIdx.x; // (token, head)
    merge_chunks<false, HD>(part + th * nslice * HD, part_ml + th * nslice * ATT_ML, att + th * HD, 1, nslice, wts,
                            wts + nslice, tot);
}

} // namespace

// ---------------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------------

struct hkhip_net {
    hkhip_engine *eng;
    hkhip_net_config cfg;
    uint32_t n_dev = 0;   // layers on the device
    bool partial = false; // only the leading layers (no embedding, final norm or output)
    uint32_t n_slots = 1, n_batch = 0, max_rows = 64, merge_max = ATT_MERGE_MAX, gqa = 0;
    bool distinct = false; // the staged pass's items each in a slot of their own
    struct Layer {
        // q, k and v rows stacked (one product, one output row per token) when the three share their
        // type; else three products into three regions of the q/k/v buffer.
        hkhip_mat wqkv{}, wq{}, wk{}, wv{}, wo{}, wgu{}, wd{};
        bool stacked = true;
        float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
        float *bqkv = nullptr;
        bool loaded = false;
    };
    std::vector<Layer> layers;
    hkhip_mat embd{}, output{};
    float *out_norm = nullptr;
    // Device buffers the network allocated, with their sizes (pass buffers: [cap tokens][...]).
    std::vector<std::pair<void *, uint64_t>> owned;
    uint32_t cap = 0; // tokens the pass buffers hold
    float *x = nullptr, *xb = nullptr, *qkv = nullptr, *att = nullptr, *h = nullptr, *part = nullptr, *part_ml = nullptr,
          *logits = nullptr, *lx = nullptr, *inv_freq = nullptr;
    uint8_t *xq = nullptr;
    __half *kc = nullptr, *vc = nullptr, *vt = nullptr; // [slot][layer][...]
    uint32_t *io = nullptr, *tok = nullptr, *pos = nullptr, *slot = nullptr; // device [tok | pos | slot][cap]
    uint32_t *att_cnt = nullptr; // [MAX_DECODE][n_heads] decode attention chunk counters (zero between launches)
    uint32_t *stage = nullptr;   // pinned host copy of io
    float *logits_h = nullptr;   // pinned host rows of hkhip_net_logits_view ([max_rows][vocab], on first use)
    // The current pass on the host: runs of consecutive positions of one sequence [begin, end).
    std::vector<std::pair<uint32_t, uint32_t>> runs;
    std::vector<uint64_t> owner; // sequence of each slot
    std::vector<uint8_t> used;
    std::map<uint32_t, hipGraphExec_t> graphs;
    std::map<uint32_t, int> shape_runs; // eager runs per decode shape (a graph is captured after one)
    uint32_t last_n = 0;
    bool last_hidden = false; // the last pass left full-network hidden states (logits rows can be read)
};

namespace {

int hfail(hipError_t e, const char *what) {
    return set_error(e == hipErrorOutOfMemory ? HKHIP_E_OUT_OF_DEVICE_MEMORY : HKHIP_E_DEVICE_FAILED, "%s: %s", what,
                     hipGetErrorString(e));
}
#define NET_TRY(expr, what)                           \
    do {                                              \
        hipError_t e_ = (expr);                       \
        if (e_ != hipSuccess) return hfail(e_, what); \
    } while (0)

uint32_t qdim(const hkhip_net_config &c) { return c.n_heads * c.head_dim; }
uint32_t kvdim(const hkhip_net_config &c) { return c.n_kv_heads * c.head_dim; }
uint32_t qkvdim(const hkhip_net_config &c) { return qdim(c) + 2 * kvdim(c); }
// Waves per decode attention workgroup (64 positions each). Two: against four, the context's loads
// spread over twice the CUs and each workgroup's dependent steps halve, while the chunks' merge
// (in the same launch) stays one round of loads up to 1024 positions: 1.614 vs 1.645 ms per token
// on Llama-3-8B shapes, 0.806 vs 0.854 on Qwen3-0.6B shapes at 512-575 positions. Eight took
// longer still than four (one CU then pulls twice the key and value bytes), and one (64 positions
// per chunk, so past 512 positions the two-round merge) 1.691 / 0.844 ms.
constexpr uint32_t ATT_DWAVES = 2;
uint32_t nslices(const hkhip_net_config &c) { return (c.max_ctx + ATT_SLICE - 1) / ATT_SLICE; }
uint32_t vt_stride(const hkhip_net_config &c) { return (c.max_ctx + 31) / 32 * 32; }
bool prefill_mfma(const hkhip_net_config &c) { return c.head_dim == 64 || c.head_dim == 128; }
uint32_t layer_count(const hkhip_net_config &c, const hkhip_net_options &o) {
    return o.layers == 0 || o.layers >= c.n_layers ? c.n_layers : o.layers;
}
uint32_t max_rows_of(const hkhip_net_options &o) { return o.n_batch ? std::min<uint32_t>(o.n_batch, 64) : 64; }
uint32_t initial_cap(const hkhip_net_options &o) {
    return std::max(std::max(o.n_batch, MAX_DECODE), max_rows_of(o));
}

// Device bytes of every buffer of a network (one function for the allocations and the estimate).
struct NetSizes {
    uint64_t cache, vtc, logits, inv_freq, part, att_cnt, lx;         // fixed
    uint64_t x, xb, qkv, att, h, xq, io;                               // for cap tokens
    uint64_t fixed() const { return 2 * cache + vtc + logits + inv_freq + part + att_cnt + lx; }
    uint64_t per_cap() const { return x + xb + qkv + att + h + xq + io; }
};
NetSizes net_sizes(const hkhip_net_config &c, uint32_t slots, uint32_t n_dev, uint32_t max_rows, uint32_t cap) {
    NetSizes z{};
    const uint64_t sl = uint64_t(slots) * n_dev, T = cap;
    z.cache = sl * c.n_kv_heads * c.max_ctx * c.head_dim * 2;
    z.vtc = sl * c.n_kv_heads * c.head_dim * vt_stride(c) * 2;
    z.logits = uint64_t(max_rows) * c.vocab * 4;
    z.inv_freq = c.rope_dim / 2 * 4 + 4;
    z.part = uint64_t(MAX_DECODE) * c.n_heads * nslices(c) * (c.head_dim + ATT_ML) * 4; // sums, then {max, sum}
    z.att_cnt = uint64_t(MAX_DECODE) * c.n_heads * ATT_CNT * 4;
    z.lx = uint64_t(max_rows) * c.dim * 4;
    const uint32_t maxk = std::max(std::max(c.dim, qdim(c)), c.ffn_dim);
    z.x = T * c.dim * 4;
    z.xb = T * std::max(c.dim, qdim(c)) * 4;
    z.qkv = T * qkvdim(c) * 4;
    z.att = T * qdim(c) * 4;
    z.h = T * c.ffn_dim * 4;
    z.xq = hkhip_act_bytes(cap, maxk);
    z.io = 3 * T * 4;
    return z;
}

int dev_alloc(hkhip_net *n, uint64_t bytes, void **p) {
    NET_TRY(hipMalloc(p, bytes ? bytes : 1), "hipMalloc");
    n->owned.push_back({*p, bytes});
    return HKHIP_OK;
}
void dev_free(hkhip_net *n, void *p) {
    if (!p) return;
    (void)hipFree(p);
    for (auto &o : n->owned)
        if (o.first == p) o = {nullptr, 0};
}

// An f32 vector of `len` floats to the device (null for an absent optional tensor).
int load_vec(hkhip_net *n, const hkhip_net_tensor &t, uint32_t len, bool optional, float **out, const char *name) {
    *out = nullptr;
    if (!t.data) {
        if (optional) return HKHIP_OK;
        return set_error(HKHIP_E_BAD_ARGUMENT, "%s is required", name);
    }
    if (t.t != HKHIP_F32 || t.bytes != uint64_t(len) * 4)
        return set_error(HKHIP_E_BAD_ARGUMENT, "%s: expected %u f32 values (type 0x00), got type 0x%02x, %llu bytes", name,
                         len, t.t, (unsigned long long)t.bytes);
    int rc = dev_alloc(n, t.bytes, reinterpret_cast<void **>(out));
    if (rc) return rc;
    return hkhip_copy_h2d(n->eng, *out, t.data, t.bytes);
}

int load_mat(hkhip_net *n, const hkhip_net_tensor &t, uint32_t rows, uint32_t cols, hkhip_mat *out, const char *name) {
    if (!t.data) return set_error(HKHIP_E_BAD_ARGUMENT, "%s is required", name);
    const int rc = hkhip_upload(n->eng, t.data, t.bytes, t.t, rows, cols, 0, out);
    if (rc) return set_error(rc, "%s (%ux%u): %s", name, rows, cols, hkhip_last_error());
    return HKHIP_OK;
}

// The q, k, v biases as one vector (zeros for an absent one); null when none is given.
int load_qkv_bias(hkhip_net *n, const hkhip_net_layer *l, uint32_t qd, uint32_t kvd, float **out) {
    *out = nullptr;
    const hkhip_net_tensor *b[3] = {&l->bq, &l->bk, &l->bv};
    const uint32_t len[3] = {qd, kvd, kvd};
    const char *name[3] = {"bq", "bk", "bv"};
    if (!b[0]->data && !b[1]->data && !b[2]->data) return HKHIP_OK;
    std::vector<float> all(qd + 2 * kvd, 0.0f);
    uint32_t off = 0;
    for (int i = 0; i < 3; i++) {
        if (b[i]->data) {
            if (b[i]->t != HKHIP_F32 || b[i]->bytes != uint64_t(len[i]) * 4)
                return set_error(HKHIP_E_BAD_ARGUMENT, "%s: expected %u f32 values (type 0x00), got type 0x%02x, %llu bytes",
                                 name[i], len[i], b[i]->t, (unsigned long long)b[i]->bytes);
            memcpy(all.data() + off, b[i]->data, b[i]->bytes);
        }
        off += len[i];
    }
    int rc = dev_alloc(n, all.size() * 4, reinterpret_cast<void **>(out));
    if (rc) return rc;
    return hkhip_copy_h2d(n->eng, *out, all.data(), all.size() * 4);
}

// Pass buffers for up to `want` tokens.
int ensure_cap(hkhip_net *n, uint32_t want) {
    if (want <= n->cap) return HKHIP_OK;
    const hkhip_net_config &c = n->cfg;
    // Freed buffers belong to captured graphs too: drop them.
    for (auto &g : n->graphs) (void)hipGraphExecDestroy(g.second);
    n->graphs.clear();
    n->shape_runs.clear();
    if (n->stage) {
        (void)hipHostFree(n->stage);
        n->stage = nullptr;
    }
    void **bufs[] = {(void **)&n->x, (void **)&n->xb, (void **)&n->qkv, (void **)&n->att, (void **)&n->h,
                     (void **)&n->xq, (void **)&n->io};
    for (void **b : bufs) {
        dev_free(n, *b);
        *b = nullptr;
    }
    const NetSizes z = net_sizes(c, n->n_slots, n->n_dev, n->max_rows, want);
    int rc;
    if ((rc = dev_alloc(n, z.x, (void **)&n->x)) || (rc = dev_alloc(n, z.xb, (void **)&n->xb)) ||
        (rc = dev_alloc(n, z.qkv, (void **)&n->qkv)) || (rc = dev_alloc(n, z.att, (void **)&n->att)) ||
        (rc = dev_alloc(n, z.h, (void **)&n->h)) || (rc = dev_alloc(n, z.xq, (void **)&n->xq)) ||
        (rc = dev_alloc(n, z.io, (void **)&n->io)))
        return rc;
    n->tok = n->io;
    n->pos = n->io + want;
    n->slot = n->io + 2 * uint64_t(want);
    NET_TRY(hipHostMalloc(reinterpret_cast<void **>(&n->stage), z.io, hipHostMallocDefault), "hipHostMalloc");
    n->cap = want;
    return HKHIP_OK;
}

// The prefill products on the quantized input already in net->xq.
int gemms(hkhip_net *net, uint32_t n, const hkhip_mat *mats, uint32_t nparts, float *const *ys, const float *const *biases,
          int mode) {
    int rc = HKHIP_OK;
    for (uint32_t i = 0; !rc && i < nparts; i++)
        rc = hkhip_mm(net->eng, &mats[i], net->xq, ys[i], n, biases ? biases[i] : nullptr, mode);
    return rc;
}
// The products of one pass. xin: f32 input [n][cols]; norm: fused RMS norm weights or null.
// Whether a product of n tokens runs quantizer + hkhip_mm (GEMM, or the small-batch MFMA kernel
// for the formats that have it) rather than the decode kernels on the f32 input: the decode
// kernels' per-token dot work grows with the token count, the small-batch kernel's does not, but
// the quantizer launches cost a few microseconds each. Measured on whole Llama-3-8B-shaped passes:
// 4 tokens 3.3 ms on the decode kernels (their 4-token form) against 4.0 on the small-batch path;
// 5, 6 and 8 tokens (the decode kernels' 8-token form) 4.9, 5.2 and 5.9 ms against 4.0-4.3.
constexpr uint32_t NET_SK_MIN = 5;
bool gemm_path(uint32_t n, int t) {
    return n > MAX_DECODE || (n >= NET_SK_MIN && (t == HKHIP_Q4_K || t == HKHIP_Q6_K));
}

// prepared: the products' Q8K input is already in net->xq (written by the attention kernel).
int product(hkhip_net *net, uint32_t n, const hkhip_mat *mats, uint32_t nparts, const float *xin, const float *norm,
            float *const *ys, const float *const *biases, int mode, bool prepared = false) {
    hkhip_engine *eng = net->eng;
    const uint32_t cols = mats[0].cols;
    if (!gemm_path(n, mats[0].t)) {
        if (norm && n > 4 && act_kind(mats[0].t) != HKHIP_ACT_F32) {
            // 5-8 tokens: the norm folded into the quantizer, then the decode kernels on the prepared
            // input (their 8-token form with the norm in the staging does not fit the registers).
            NET_TRY(launch_qact_row(xin, n, cols, act_kind(mats[0].t), net->xq, norm, net->cfg.rms_eps, eng->cur),
                    "rmsnorm + qact");
            return hkhip_matvec_parts(eng, mats, nparts, nullptr, net->xq, n, ys, biases, mode);
        }
        if (norm) {
            const int rc = hkhip_matvec_parts_rmsnorm(eng, mats, nparts, xin, norm, net->cfg.rms_eps, n, ys, biases, mode);
            if (rc != HKHIP_E_UNSUPPORTED_SHAPE) return rc;
            hipLaunchKernelGGL(rmsnorm_kernel, dim3(n), dim3(256), 0, eng->cur, xin, norm, net->xb, cols, net->cfg.rms_eps);
            NET_TRY(hipGetLastError(), "rmsnorm");
            xin = net->xb;
        }
        return hkhip_matvec_parts(eng, mats, nparts, xin, nullptr, n, ys, biases, mode);
    }
    if (norm && act_kind(mats[0].t) != HKHIP_ACT_F32) { // the norm folded into the quantizer
        NET_TRY(launch_qact_row(xin, n, cols, act_kind(mats[0].t), net->xq, norm, net->cfg.rms_eps, eng->cur),
                "rmsnorm + qact");
        return gemms(net, n, mats, nparts, ys, biases, mode);
    }
    if (norm) {
        hipLaunchKernelGGL(rmsnorm_kernel, dim3(n), dim3(256), 0, eng->cur, xin, norm, net->xb, cols, net->cfg.rms_eps);
        NET_TRY(hipGetLastError(), "rmsnorm");
        xin = net->xb;
    }
    if (act_kind(mats[0].t) == HKHIP_ACT_F32) { // dotted against the f32 input: passes of 8 tokens
        int rc = HKHIP_OK;
        for (uint32_t t0 = 0; !rc && t0 < n; t0 += MAX_DECODE) {
            const uint32_t nc = n - t0 < MAX_DECODE ? n - t0 : MAX_DECODE;
            float *yc[4];
            for (uint32_t i = 0; i < nparts; i++)
                yc[i] = ys[i] + uint64_t(t0) * (mode == HKHIP_SILU_MUL ? mats[i].rows / 2 : mats[i].rows);
            rc = hkhip_matvec_parts(eng, mats, nparts, xin + uint64_t(t0) * cols, nullptr, nc, yc, biases, mode);
        }
        return rc;
    }
    const int rc = prepared ? HKHIP_OK : hkhip_qact(eng, xin, n, cols, act_kind(mats[0].t), net->xq);
    return rc ? rc : gemms(net, n, mats, nparts, ys, biases, mode);
}

// Query heads per workgroup of the grouped attention kernel: the largest divisor of the GQA group
// size up to 8 (the MFMA tile's hi / lo column halves).
uint32_t group_block(const hkhip_net_config &c) {
    const uint32_t grp = c.n_heads / c.n_kv_heads;
    uint32_t ng = 8;
    while (grp % ng) ng--;
    return ng;
}

// Whether nt tokens' decode attention over gb chunks runs on the grouped MFMA kernel
// (attn_decode_gqa_kernel). By size: once the per-head kernel's waves (2 gb heads nt, two per
// chunk) pass 2048, one round at its ~180 registers (two waves per SIMD), where it was measured
// to fall behind:
// per Llama-3-8B-shaped layer (32 / 8 heads), 8 tokens at 800 positions 23.3 vs 17.4 us, at 1600
// 44.0 vs 30.5, at 3000 97.6 vs 50.3; below, the per-head kernel is as fast or up to 2 us faster
// (8 tokens at <= 128 positions 7.2 vs 8.6, 2 tokens at 800 10.3 vs 12.6; Qwen3-0.6B-shaped,
// 16 / 8 heads: 8 tokens at 800 14.1 vs 15.4, at 1600 27.4 vs 24.4).
// q8: the o product would take the results as a Q8K input (attn_quantize_block); when a head block
// is whole Q8K blocks the grouped kernel then also saves the quantizer launch (4.6-4.8 us), which
// outweighs what the per-head kernel is faster by at any size measured above.
bool q8_in_attention(const hkhip_net *net, uint32_t gb) {
    const hkhip_net_config &c = net->cfg;
    return group_block(c) * c.head_dim % QK_K == 0 && (gb == 1 || gb <= net->merge_max);
}
bool grouped_attention(const hkhip_net *net, uint32_t nt, uint32_t gb, bool q8 = false) {
    const hkhip_net_config &c = net->cfg;
    if (net->gqa == 2 || (c.head_dim != 64 && c.head_dim != 128)) return false;
    return net->gqa == 1 || uint64_t(2) * gb * c.n_heads * nt > 2048 || (q8 && q8_in_attention(net, gb));
}

// Decode attention over tokens [t0, t0 + nt) of the pass (nt <= MAX_DECODE), gb chunks per
// (head, token). fused: a one-token pass whose attention kernel also does the head norms, the
// rotation and the cache writes (ra's fields).
int decode_attention(hkhip_net *net, const RopeArgs &ra, const __half *kc, const __half *vc, uint32_t t0, uint32_t nt,
                     uint32_t gb, bool fused, bool *q8_done = nullptr) {
    const hkhip_net_config &c = net->cfg;
    hipStream_t s = net->eng->cur;
    AttnArgs aa{ra.q + uint64_t(t0) * ra.sq, kc, vc, net->part, net->pos + t0, net->slot + t0, ra.kv_slot, nt,
                c.n_heads, c.n_kv_heads, c.head_dim, c.max_ctx, 1.0f / sqrtf(float(c.head_dim)), ra.sq};
    float *att = net->att + uint64_t(t0) * qdim(c);
    aa.att = gb == 1 ? att : nullptr;
    aa.fused = fused ? 1 : 0;
    aa.r = ra;
    const bool merge_in = gb > 1 && gb <= net->merge_max;
    aa.cnt = merge_in ? net->att_cnt : nullptr;
    aa.merge_out = att;
    aa.part_ml = net->part_ml;
    // The per-head kernel (G = 1) or, past one round of its waves, the grouped MFMA kernel (see
    // grouped_attention). The per-head kernel's FMA form with G = the group size measured slower
    // (a wave runs the group's dots, softmax and value sums one after another: 23.1 vs 9.8 us per
    // Llama-3-8B layer at positions 512-575, G = 4).
    constexpr int NV = int(ATT_DWAVES);
    if (grouped_attention(net, nt, gb, q8_done && t0 == 0)) { // fused: every token in its own slot
        const uint32_t ng = group_block(c);
        const dim3 gg(gb, c.n_heads / ng, nt);
        // q8_done (a pass's only attention launch, the o product on a Q8K input): the workgroups
        // that write the results also quantize them, when a head block is whole Q8K blocks and no
        // separate merge kernel follows; the caller then skips the o product's quantizer launch.
        if (q8_done && t0 == 0 && q8_in_attention(net, gb)) {
            aa.q8_on = 1;
            aa.q8 = q8k_planes(reinterpret_cast<uint8_t *>(net->xq), act_layout(nt, qdim(c)), nt, qdim(c));
            *q8_done = true;
        }
        // The fused form runs four waves of 32 positions per chunk: with two of 64 the q rows'
        // registers next to the rows in flight left one wave per SIMD (233 VGPRs + 32 AGPRs).
        if (c.head_dim == 64 && fused)
            hipLaunchKernelGGL((attn_decode_gqa_kernel<64, 2 * NV, 1, true>), gg, dim3(128 * NV), 0, s, aa, ng);
        else if (c.head_dim == 64)
            hipLaunchKernelGGL((attn_decode_gqa_kernel<64, NV, 2, false>), gg, dim3(64 * NV), 0, s, aa, ng);
        else if (fused)
            hipLaunchKernelGGL((attn_decode_gqa_kernel<128, 2 * NV, 1, true>), gg, dim3(128 * NV), 0, s, aa, ng);
        else
            hipLaunchKernelGGL((attn_decode_gqa_kernel<128, NV, 2, false>), gg, dim3(64 * NV), 0, s, aa, ng);
    } else {
    const dim3 dg(gb, c.n_heads, nt), db(64 * ATT_DWAVES);
    if (c.head_dim == 64)
        hipLaunchKernelGGL((attn_decode_kernel<64, NV, 1>), dg, db, 0, s, aa);
    else if (c.head_dim == 128)
        hipLaunchKernelGGL((attn_decode_kernel<128, NV, 1>), dg, db, 0, s, aa);
    else
        hipLaunchKernelGGL((attn_decode_kernel<256, NV, 1>), dg, db, 0, s, aa);
    }
    NET_TRY(hipGetLastError(), "decode attention");
    if (gb > 1 && !merge_in) {
        const dim3 cg(c.n_heads, nt), cb(256);
        if (c.head_dim == 64)
            hipLaunchKernelGGL(attn_combine_kernel<64>, cg, cb, gb * 8, s, net->part, net->part_ml, att, c.n_heads, gb);
        else if (c.head_dim == 128)
            hipLaunchKernelGGL(attn_combine_kernel<128>, cg, cb, gb * 8, s, net->part, net->part_ml, att, c.n_heads, gb);
        else
            hipLaunchKernelGGL(attn_combine_kernel<256>, cg, cb, gb * 8, s, net->part, net->part_ml, att, c.n_heads, gb);
        NET_TRY(hipGetLastError(), "decode attention combine");
    }
    return HKHIP_OK;
}

// One pass over the device layers for the n tokens whose tokens / positions / slots are in net->io
// (and, for a partial network, whose hidden states are in net->x). gb: decode attention chunks per
// (head, token). lg: also the logits of the last token into net->logits.
int run_pass(hkhip_net *net, uint32_t n, uint32_t gb, bool lg) {
    const hkhip_net_config &c = net->cfg;
    hkhip_engine *eng = net->eng;
    hipStream_t s = eng->cur;
    int rc;
    if (!net->partial)
        NET_TRY(launch_dequant_gather(net->embd.t, reinterpret_cast<const uint8_t *>(net->embd.mem), net->embd.rows,
                                      c.dim, net->tok, n, net->x, s), "embedding");
    const uint64_t cache_layer = uint64_t(c.n_kv_heads) * c.max_ctx * c.head_dim;
    const uint64_t vt_layer = uint64_t(c.n_kv_heads) * c.head_dim * vt_stride(c);
    for (uint32_t li = 0; li < net->n_dev; li++) {
        const hkhip_net::Layer &L = net->layers[li];
        {
            if (L.stacked) {
                float *const ys[1] = {net->qkv};
                const float *const bs[1] = {L.bqkv};
                if ((rc = product(net, n, &L.wqkv, 1, net->x, L.attn_norm, ys, bs, HKHIP_STORE))) return rc;
            } else {
                const hkhip_mat *ms[3] = {&L.wq, &L.wk, &L.wv};
                float *const out[3] = {net->qkv, net->qkv + uint64_t(net->cap) * qdim(c),
                                       net->qkv + uint64_t(net->cap) * (qdim(c) + kvdim(c))};
                const uint32_t boff[3] = {0, qdim(c), qdim(c) + kvdim(c)};
                for (int i = 0; i < 3; i++) {
                    float *const ys[1] = {out[i]};
                    const float *const bs[1] = {L.bqkv ? L.bqkv + boff[i] : nullptr};
                    if ((rc = product(net, n, ms[i], 1, net->x, L.attn_norm, ys, bs, HKHIP_STORE))) return rc;
                }
            }
        }
        // Rows of q, k, v: stride S (stacked) or their own regions of the buffer (qd, kvd).
        float *const q = net->qkv;
        float *const k = L.stacked ? q + qdim(c) : q + uint64_t(net->cap) * qdim(c);
        float *const v = L.stacked ? k + kvdim(c) : k + uint64_t(net->cap) * kvdim(c);
        const uint32_t S = L.stacked ? qkvdim(c) : qdim(c), SKV = L.stacked ? qkvdim(c) : kvdim(c);
        __half *const kc = net->kc + li * cache_layer, *const vc = net->vc + li * cache_layer;
        __half *const vtl = net->vt + li * vt_layer;
        RopeArgs ra{q, k, v, L.q_norm, L.k_norm, net->inv_freq, kc, vc, vtl, net->pos, net->slot,
                    uint64_t(net->n_dev) * cache_layer, uint64_t(net->n_dev) * vt_layer, c.n_heads, c.n_kv_heads,
                    c.head_dim, c.rope_dim / 2, c.rope_neox, c.max_ctx, vt_stride(c), S, SKV, 0, c.rope_mscale,
                    c.rms_eps};
        // Prefill passes write the value heads with v_cache_block (coalesced transposed writes).
        // Decode passes: the o product may take its Q8K input from the attention kernel, and the
        // attention kernel does the rope / cache work itself when every token has a slot of its own
        // (no token then reads another's new row). For the per-head kernel that was first one-token
        // passes only; 2-4 sequences per pass fused measured 1.3-1.8 us per Llama-3-8B-shaped layer
        // below the separate rope launch.
        const bool vsep = n > MAX_DECODE;
        const bool want_q8 = !vsep && gemm_path(n, L.wo.t) && act_kind(L.wo.t) == HKHIP_ACT_Q8K;
        // (The grouped kernel rotates q in its operand registers: neox pairs must lie 32 dimensions
        // apart or a multiple of it.)
        const bool rope_in_lanes = !c.rope_neox || c.rope_dim / 2 % 32 == 0;
        const bool fused = !vsep && net->distinct && (!grouped_attention(net, n, gb, want_q8) || rope_in_lanes);
        ra.nheads = c.n_heads + (vsep ? 1 : 2) * c.n_kv_heads;
        if (vsep) { // one launch: rope / key writes, then the value rows
            ra.ntok = n;
            const uint32_t rx = (ra.nheads + 3) / 4;
            hipLaunchKernelGGL(rope_kv_v_kernel, dim3(rx * n + c.n_kv_heads * ((n + 15) / 16)), dim3(256), 0, s, ra, v, rx);
            NET_TRY(hipGetLastError(), "rope / kv write");
        } else if (!fused) {
            hipLaunchKernelGGL(rope_kv_kernel, dim3((ra.nheads + 3) / 4, n), dim3(256), 0, s, ra);
            NET_TRY(hipGetLastError(), "rope / kv write");
        }
        bool att_q8 = false;
        if (n <= MAX_DECODE) {
            if ((rc = decode_attention(net, ra, kc, vc, 0, n, gb, fused, want_q8 ? &att_q8 : nullptr))) return rc;
        } else {
            // Each sequence's run of consecutive positions: longer than a decode pass on the MFMA
            // prefill kernel, else (and for head dims it does not take) on the decode kernel, up to
            // MAX_DECODE tokens per launch.
            for (const auto &r : net->runs) {
                const uint32_t len = r.second - r.first;
                if (len > MAX_DECODE && prefill_mfma(c)) {
                    AttnPArgs pa{q + uint64_t(r.first) * S, kc, vtl, net->att + uint64_t(r.first) * qdim(c),
                                 net->pos + r.first, net->slot + r.first, ra.kv_slot, ra.vt_slot, len, c.n_heads,
                                 c.n_kv_heads, c.max_ctx, vt_stride(c), 1.0f / sqrtf(float(c.head_dim)), S};
                    const dim3 pg((len + 31) / 32 * c.n_heads);
                    // Four waves: eight per workgroup (two per SIMD, the key tiles split eight ways)
                    // measured 21.3 vs 18.4 us per Llama-3-8B layer and 15.2 vs 16.4 us per Qwen3-0.6B layer.
                    const hipError_t ae = c.head_dim == 64 ? launch_attn_prefill<64, 4>(pg, pa, s)
                                                           : launch_attn_prefill<128, 4>(pg, pa, s);
                    NET_TRY(ae, "prefill attention");
                } else {
                    for (uint32_t t0 = r.first; t0 < r.second; t0 += MAX_DECODE)
                        if ((rc = decode_attention(net, ra, kc, vc, t0, std::min(MAX_DECODE, r.second - t0), gb, false)))
                            return rc;
                }
            }
        }
        {
            float *const ys[1] = {net->x};
            if ((rc = product(net, n, &L.wo, 1, net->att, nullptr, ys, nullptr, HKHIP_ACCUMULATE, att_q8))) return rc;
        }
        { // gate/up with silu(gate) * up in the products' epilogue (decode kernels and GEMMs alike)
            float *const ys[1] = {net->h};
            if ((rc = product(net, n, &L.wgu, 1, net->x, L.ffn_norm, ys, nullptr, HKHIP_SILU_MUL))) return rc;
        }
        {
            float *const ys[1] = {net->x};
            if ((rc = product(net, n, &L.wd, 1, net->h, nullptr, ys, nullptr, HKHIP_ACCUMULATE))) return rc;
        }
    }
    if (!lg) return HKHIP_OK;
    // Logits of the last token (cpu_backend.zig:324-331 logitsFor).
    float *const ys[1] = {net->logits};
    return product(net, 1, &net->output, 1, net->x + uint64_t(n - 1) * c.dim, net->out_norm, ys, nullptr, HKHIP_STORE);
}

// Checks a pass's items, assigns slots (engine.zig:556-568 slotFor) and stages tokens, positions
// and slots in net->io; fills net->runs. Returns the largest position.
int stage_items(hkhip_net *net, const hkhip_item *items, uint32_t n, uint32_t *max_pos) {
    const hkhip_net_config &c = net->cfg;
    if (net->n_batch && n > net->n_batch) return set_error(HKHIP_E_BAD_ARGUMENT, "%u items: n_batch is %u", n, net->n_batch);
    for (uint32_t i = 0; i < n; i++) {
        if (items[i].pos >= c.max_ctx)
            return set_error(HKHIP_E_CONTEXT_FULL, "item %u: position %u, max_ctx %u", i, items[i].pos, c.max_ctx);
        if (!net->partial && items[i].token >= c.vocab)
            return set_error(HKHIP_E_BAD_ARGUMENT, "item %u: token %u >= vocab %u", i, items[i].token, c.vocab);
    }
    // Slots: the sequence's own, else a free one; positions of a sequence increase through the pass.
    std::vector<uint32_t> sl(n);
    std::vector<int64_t> last(net->n_slots, -1);
    std::vector<uint8_t> used = net->used;
    std::vector<uint64_t> owner = net->owner;
    for (uint32_t i = 0; i < n; i++) {
        uint32_t s = UINT32_MAX;
        for (uint32_t j = 0; j < net->n_slots && s == UINT32_MAX; j++)
            if (used[j] && owner[j] == items[i].seq) s = j;
        for (uint32_t j = 0; j < net->n_slots && s == UINT32_MAX; j++)
            if (!used[j]) {
                used[j] = 1;
                owner[j] = items[i].seq;
                s = j;
            }
        if (s == UINT32_MAX)
            return set_error(HKHIP_E_NO_SLOT, "item %u: all %u cache slots are held by other sequences", i, net->n_slots);
        if (int64_t(items[i].pos) <= last[s])
            return set_error(HKHIP_E_BAD_ARGUMENT, "item %u: position %u of sequence %llu after position %lld", i,
                             items[i].pos, (unsigned long long)items[i].seq, (long long)last[s]);
        last[s] = items[i].pos;
        sl[i] = s;
    }
    int rc;
    if ((rc = ensure_cap(net, n))) return rc;
    net->used = used;
    net->owner = owner;
    uint32_t mp = 0;
    net->runs.clear();
    for (uint32_t i = 0; i < n; i++) {
        net->stage[i] = items[i].token;
        net->stage[net->cap + i] = items[i].pos;
        net->stage[2 * net->cap + i] = sl[i];
        mp = std::max(mp, items[i].pos);
        if (i && sl[i] == sl[i - 1] && items[i].pos == items[i - 1].pos + 1)
            net->runs.back().second = i + 1;
        else
            net->runs.push_back({i, i + 1});
    }
    *max_pos = mp;
    net->distinct = true; // every item in a slot of its own
    std::vector<uint8_t> seen(net->n_slots, 0);
    for (uint32_t i = 0; i < n && net->distinct; i++) {
        if (seen[sl[i]]) net->distinct = false;
        seen[sl[i]] = 1;
    }
    NET_TRY(hipMemcpyAsync(net->io, net->stage, uint64_t(3) * net->cap * 4, hipMemcpyHostToDevice, net->eng->cur),
            "items");
    return HKHIP_OK;
}

int check_loaded(const hkhip_net *net) {
    if (!net->partial && (!net->embd.mem || !net->output.mem))
        return set_error(HKHIP_E_BAD_ARGUMENT, "tok_embd / output not loaded");
    for (const auto &L : net->layers)
        if (!L.loaded) return set_error(HKHIP_E_BAD_ARGUMENT, "a layer is not loaded");
    return HKHIP_OK;
}

// A pass over n staged items (hidden states already in net->x for a partial network); the pass is
// done when this returns (the next call reuses the pinned staging buffer).
int forward_staged(hkhip_net *net, uint32_t n, uint32_t max_pos, bool lg) {
    const hkhip_net_config &c = net->cfg;
    hipStream_t s = net->eng->cur;
    int rc;
    // Decode attention chunks: as many as cover positions 0..max_pos (ATT_DWAVES waves of 64
    // positions each), so that short contexts skip the merge; one graph per (size, chunks, whether
    // every item has a slot of its own: the fused attention), so a
    // growing context captures a new graph every 128 positions. (Rounding the count up to a power of
    // two, for fewer graphs, launched up to 3 empty chunks per (head, token) at 512-575 positions:
    // 1.632 vs 1.626 ms per Llama-3-8B token, 0.838 vs 0.823 ms per Qwen3-0.6B token, 3.18 vs 3.12 ms
    // per 8-sequence pass with its logits.)
    const uint32_t dw = ATT_DWAVES, gmax = (nslices(c) + dw - 1) / dw, need = (max_pos + 64 * dw) / (64 * dw);
    const uint32_t gb = std::min(need, gmax);
    if (n > MAX_DECODE) { // prefill: run directly
        if ((rc = run_pass(net, n, gb, lg))) return rc;
        NET_TRY(hipStreamSynchronize(s), "prefill pass");
        return HKHIP_OK;
    }
    const uint32_t key = n | (gb << 8) | (net->distinct ? 1u << 30 : 0u) | (lg ? 1u << 31 : 0u);
    auto it = net->graphs.find(key);
    if (it != net->graphs.end()) {
        NET_TRY(hipGraphLaunch(it->second, s), "graph launch");
    } else if (net->shape_runs[key]++ == 0) {
        if ((rc = run_pass(net, n, gb, lg))) return rc; // first pass of this shape: eager (fills the launch caches)
    } else {
        hipGraph_t g = nullptr;
        NET_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture");
        rc = run_pass(net, n, gb, lg);
        const hipError_t e = hipStreamEndCapture(s, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        NET_TRY(e, "end capture");
        hipGraphExec_t ex = nullptr;
        const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        NET_TRY(ei, "graph instantiate");
        net->graphs[key] = ex;
        NET_TRY(hipGraphLaunch(ex, s), "graph launch");
    }
    NET_TRY(hipStreamSynchronize(s), "pass");
    return HKHIP_OK;
}

int forward_items(hkhip_net *net, const hkhip_item *items, uint32_t n, bool lg) {
    if (!net || (n && !items)) return set_error(HKHIP_E_BAD_ARGUMENT, "null argument");
    if (net->partial) return set_error(HKHIP_E_PARTIAL, "a partial network runs hkhip_net_forward_partial");
    if (n == 0) return HKHIP_OK;
    int rc;
    if ((rc = check_loaded(net))) return rc;
    if (hipSetDevice(net->eng->device) != hipSuccess) return set_error(HKHIP_E_DEVICE_FAILED, "hipSetDevice");
    uint32_t max_pos = 0;
    net->last_n = 0;
    net->last_hidden = false;
    if ((rc = stage_items(net, items, n, &max_pos)) || (rc = forward_staged(net, n, max_pos, lg))) return rc;
    net->last_n = n;
    net->last_hidden = true;
    return HKHIP_OK;
}

// Device bytes of one layer's tensors as the network holds them (stacked q/k/v or three matrices,
// interleaved gate/up, f32 vectors, the stacked bias); 0 when a matrix type has no kernel.
uint64_t layer_dev_bytes(const hkhip_net_config &c, const hkhip_net_layer &l) {
    const uint32_t qd = qdim(c), kvd = kvdim(c);
    auto mat = [&](uint8_t t, uint32_t rows, uint32_t cols) -> uint64_t {
        if (!block_elems(t) || cols % block_elems(t)) return 0;
        return weight_layout(t, rows, cols).total;
    };
    uint64_t total = 2 * uint64_t(c.dim) * 4;
    if (l.q_norm.data) total += uint64_t(c.head_dim) * 4;
    if (l.k_norm.data) total += uint64_t(c.head_dim) * 4;
    if (l.bq.data || l.bk.data || l.bv.data) total += uint64_t(qd + 2 * kvd) * 4;
    uint64_t m[4];
    if (l.wq.t == l.wk.t && l.wq.t == l.wv.t) {
        m[0] = mat(l.wq.t, qd + 2 * kvd, c.dim);
        if (!m[0]) return 0;
        total += m[0];
    } else {
        m[0] = mat(l.wq.t, qd, c.dim);
        m[1] = mat(l.wk.t, kvd, c.dim);
        m[2] = mat(l.wv.t, kvd, c.dim);
        if (!m[0] || !m[1] || !m[2]) return 0;
        total += m[0] + m[1] + m[2];
    }
    m[0] = mat(l.wo.t, c.dim, qd);
    m[1] = mat(l.w_gate.t, 2 * c.ffn_dim, c.dim);
    m[2] = mat(l.w_down.t, c.dim, c.ffn_dim);
    if (!m[0] || !m[1] || !m[2]) return 0;
    return total + m[0] + m[1] + m[2];
}

// A shape the network takes (max_ctx 0 too: the planner's base estimate, backend.zig:92-126).
bool config_ok(const hkhip_net_config &c) {
    return c.dim && c.n_layers && c.n_heads && c.n_kv_heads && !(c.n_heads % c.n_kv_heads) && c.ffn_dim && c.vocab &&
           (c.head_dim == 64 || c.head_dim == 128 || c.head_dim == 256) && !(c.rope_dim % 2) &&
           c.rope_dim <= c.head_dim;
}

} // namespace

extern "C" {

int hkhip_net_create_opts(hkhip_engine *eng, const hkhip_net_config *cfg, const hkhip_net_options *opts, hkhip_net **out) {
    if (!eng || !cfg || !out) return set_error(HKHIP_E_BAD_ARGUMENT, "null argument");
    *out = nullptr;
    const hkhip_net_config &c = *cfg;
    const hkhip_net_options o = opts ? *opts : hkhip_net_options{};
    if (!c.dim || !c.n_layers || !c.n_heads || !c.n_kv_heads || c.n_heads % c.n_kv_heads || !c.ffn_dim || !c.vocab ||
        !c.max_ctx)
        return set_error(HKHIP_E_BAD_ARGUMENT, "bad network shape");
    if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256)
        return set_error(HKHIP_E_UNSUPPORTED_SHAPE, "head_dim %u: 64, 128 or 256", c.head_dim);
    if (c.rope_dim % 2 || c.rope_dim > c.head_dim) return set_error(HKHIP_E_BAD_ARGUMENT, "rope_dim %u", c.rope_dim);
    if (hipSetDevice(eng->device) != hipSuccess) return set_error(HKHIP_E_DEVICE_FAILED, "hipSetDevice");
    hkhip_net *n = new hkhip_net();
    n->eng = eng;
    n->cfg = c;
    n->n_dev = layer_count(c, o);
    n->partial = n->n_dev < c.n_layers;
    n->n_slots = o.slots ? o.slots : 1;
    n->n_batch = o.n_batch;
    n->max_rows = max_rows_of(o);
    n->merge_max = o.attn_merge_max ? std::min(o.attn_merge_max, ATT_MERGE_MAX) : ATT_MERGE_MAX;
    if (o.attn_gqa > 2) {
        delete n;
        return set_error(HKHIP_E_BAD_ARGUMENT, "attn_gqa %u: 0, 1 or 2", o.attn_gqa);
    }
    n->gqa = o.attn_gqa;
    n->layers.resize(n->n_dev);
    n->owner.assign(n->n_slots, 0);
    n->used.assign(n->n_slots, 0);
    int rc = HKHIP_OK;
    const NetSizes z = net_sizes(c, n->n_slots, n->n_dev, n->max_rows, 0);
    if ((rc = dev_alloc(n, z.cache, (void **)&n->kc)) || (rc = dev_alloc(n, z.cache, (void **)&n->vc)) ||
        (rc = dev_alloc(n, z.vtc, (void **)&n->vt)) || (rc = dev_alloc(n, z.logits, (void **)&n->logits)) ||
        (rc = dev_alloc(n, z.inv_freq, (void **)&n->inv_freq)) || (rc = dev_alloc(n, z.part, (void **)&n->part)) ||
        (rc = dev_alloc(n, z.att_cnt, (void **)&n->att_cnt)) || (rc = dev_alloc(n, z.lx, (void **)&n->lx)) ||
        (rc = ensure_cap(n, initial_cap(o)))) {
        hkhip_net_destroy(n);
        return rc;
    }
    // The chunk partials' {max, sum} pairs follow their sums: [8][heads][chunks][hd], then [..][2].
    n->part_ml = n->part + uint64_t(MAX_DECODE) * c.n_heads * nslices(c) * c.head_dim;
    // Positions a pass has not written yet are read (and weighted by 0) by the attention kernels:
    // they must hold finite values. The chunk counters start at zero.
    if (hipMemset(n->kc, 0, z.cache) != hipSuccess || hipMemset(n->vc, 0, z.cache) != hipSuccess ||
        hipMemset(n->vt, 0, z.vtc) != hipSuccess || hipMemset(n->att_cnt, 0, z.att_cnt) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        hkhip_net_destroy(n);
        return set_error(HKHIP_E_DEVICE_FAILED, "clearing the caches");
    }
    // The caller's inverse frequencies (hk computes them with any scaling on the host), or
    // ropeInvFreq without scaling (ops.zig:96-146): base^(-2i/n_rot) in f64, then f32.
    std::vector<float> f(c.rope_dim / 2 + 1, 0.0f);
    for (uint32_t i = 0; i < c.rope_dim / 2; i++)
        f[i] = c.inv_freq ? c.inv_freq[i] : float(pow(double(c.rope_base), -double(2 * i) / double(c.rope_dim)));
    n->cfg.inv_freq = nullptr; // the caller's array is not kept
    for (uint32_t i = 0; i < c.rope_dim / 2; i++)
        if (!(f[i] > 0.0f) || !std::isfinite(f[i])) {
            hkhip_net_destroy(n);
            return set_error(HKHIP_E_BAD_ARGUMENT, "inv_freq[%u] = %g: expected a positive number", i, double(f[i]));
        }
    if (!(n->cfg.rope_mscale > 0.0f)) n->cfg.rope_mscale = 1.0f;
    if ((rc = hkhip_copy_h2d(eng, n->inv_freq, f.data(), f.size() * 4))) {
        hkhip_net_destroy(n);
        return rc;
    }
    *out = n;
    return HKHIP_OK;
}

int hkhip_net_create(hkhip_engine *eng, const hkhip_net_config *cfg, hkhip_net **out) {
    return hkhip_net_create_opts(eng, cfg, nullptr, out);
}

void hkhip_net_destroy(hkhip_net *net) {
    if (!net) return;
    (void)hipSetDevice(net->eng->device);
    (void)hipStreamSynchronize(net->eng->cur);
    for (auto &g : net->graphs) (void)hipGraphExecDestroy(g.second);
    for (auto &L : net->layers) {
        hkhip_mat *ms[] = {&L.wqkv, &L.wq, &L.wk, &L.wv, &L.wo, &L.wgu, &L.wd};
        for (hkhip_mat *m : ms) hkhip_free(net->eng, m);
    }
    hkhip_free(net->eng, &net->embd);
    hkhip_free(net->eng, &net->output);
    for (auto &p : net->owned)
        if (p.first) (void)hipFree(p.first);
    if (net->stage) (void)hipHostFree(net->stage);
    if (net->logits_h) (void)hipHostFree(net->logits_h);
    delete net;
}

int hkhip_net_load_layer(hkhip_net *net, uint32_t li, const hkhip_net_layer *l) {
    if (!net || !l) return set_error(HKHIP_E_BAD_ARGUMENT, "null argument");
    const hkhip_net_config &c = net->cfg;
    if (li >= net->n_dev)
        return set_error(HKHIP_E_BAD_ARGUMENT, "layer %u: the network holds layers 0..%u", li, net->n_dev - 1);
    hkhip_net::Layer &L = net->layers[li];
    if (L.loaded) return set_error(HKHIP_E_BAD_ARGUMENT, "layer %u is already loaded", li);
    const uint32_t qd = qdim(c), kvd = kvdim(c);
    int rc;
    if ((rc = load_vec(net, l->attn_norm, c.dim, false, &L.attn_norm, "attn_norm")) ||
        (rc = load_vec(net, l->ffn_norm, c.dim, false, &L.ffn_norm, "ffn_norm")) ||
        (rc = load_vec(net, l->q_norm, c.head_dim, true, &L.q_norm, "q_norm")) ||
        (rc = load_vec(net, l->k_norm, c.head_dim, true, &L.k_norm, "k_norm")) ||
        (rc = load_qkv_bias(net, l, qd, kvd, &L.bqkv)))
        return rc;
    if (l->w_gate.t != l->w_up.t) return set_error(HKHIP_E_BAD_ARGUMENT, "w_gate and w_up must share their type");
    if ((rc = load_mat(net, l->wo, c.dim, qd, &L.wo, "wo")) || (rc = load_mat(net, l->w_down, c.dim, c.ffn_dim, &L.wd, "w_down")))
        return rc;
    L.stacked = l->wq.t == l->wk.t && l->wq.t == l->wv.t;
    if (!L.stacked) {
        if ((rc = load_mat(net, l->wq, qd, c.dim, &L.wq, "wq")) || (rc = load_mat(net, l->wk, kvd, c.dim, &L.wk, "wk")) ||
            (rc = load_mat(net, l->wv, kvd, c.dim, &L.wv, "wv")))
            return rc;
    } else {
        // q, k and v rows stacked into one matrix (one product launch, one output row per token).
        const int64_t qb = hkhip_matrix_bytes(l->wq.t, 1, c.dim);
        if (qb < 0) return int(qb);
        const hkhip_net_tensor *parts[3] = {&l->wq, &l->wk, &l->wv};
        const uint32_t prow[3] = {qd, kvd, kvd};
        const char *pname[3] = {"wq", "wk", "wv"};
        std::vector<uint8_t> qkv(uint64_t(qb) * (qd + 2 * kvd));
        uint64_t off = 0;
        for (int i = 0; i < 3; i++) {
            const uint64_t want = uint64_t(qb) * prow[i];
            if (!parts[i]->data || parts[i]->bytes != want)
                return set_error(HKHIP_E_BAD_ARGUMENT, "%s: expected %llu bytes", pname[i], (unsigned long long)want);
            memcpy(qkv.data() + off, parts[i]->data, want);
            off += want;
        }
        const hkhip_net_tensor t{qkv.data(), qkv.size(), l->wq.t};
        if ((rc = load_mat(net, t, qd + 2 * kvd, c.dim, &L.wqkv, "wq/wk/wv"))) return rc;
    }
    // Gate and up rows interleaved (row 2i = gate i, 2i + 1 = up i) for the fused silu(gate)*up.
    const int64_t rb = hkhip_matrix_bytes(l->w_gate.t, 1, c.dim);
    if (rb < 0) return int(rb);
    if (!l->w_gate.data || !l->w_up.data || l->w_gate.bytes != uint64_t(rb) * c.ffn_dim || l->w_up.bytes != l->w_gate.bytes)
        return set_error(HKHIP_E_BAD_ARGUMENT, "w_gate / w_up: expected %llu bytes each",
                         (unsigned long long)(uint64_t(rb) * c.ffn_dim));
    std::vector<uint8_t> inter(uint64_t(rb) * 2 * c.ffn_dim);
    const uint8_t *g = static_cast<const uint8_t *>(l->w_gate.data), *u = static_cast<const uint8_t *>(l->w_up.data);
    for (uint32_t i = 0; i < c.ffn_dim; i++) {
        memcpy(&inter[(2 * uint64_t(i)) * rb], g + uint64_t(i) * rb, size_t(rb));
        memcpy(&inter[(2 * uint64_t(i) + 1) * rb], u + uint64_t(i) * rb, size_t(rb));
    }
    const hkhip_net_tensor gu{inter.data(), inter.size(), l->w_gate.t};
    if ((rc = load_mat(net, gu, 2 * c.ffn_dim, c.dim, &L.wgu, "w_gate/w_up"))) return rc;
    L.loaded = true;
    return HKHIP_OK;
}

int hkhip_net_load_io(hkhip_net *net, hkhip_net_tensor tok_embd, hkhip_net_tensor out_norm, hkhip_net_tensor output) {
    if (!net) return set_error(HKHIP_E_BAD_ARGUMENT, "null network");
    if (net->partial) return set_error(HKHIP_E_PARTIAL, "a partial network has no embedding or output");
    const hkhip_net_config &c = net->cfg;
    if (net->embd.mem || net->output.mem) return set_error(HKHIP_E_BAD_ARGUMENT, "tok_embd / output are already loaded");
    int rc;
    if ((rc = load_mat(net, tok_embd, c.vocab, c.dim, &net->embd, "tok_embd")) ||
        (rc = load_vec(net, out_norm, c.dim, false, &net->out_norm, "out_norm")) ||
        (rc = load_mat(net, output, c.vocab, c.dim, &net->output, "output")))
        return rc;
    return HKHIP_OK;
}

int hkhip_net_forward_items(hkhip_net *net, const hkhip_item *items, uint32_t n) {
    return forward_items(net, items, n, false);
}

int hkhip_net_forward_partial(hkhip_net *net, const hkhip_item *items, uint32_t n, float *hidden_host) {
    if (!net || (n && (!items || !hidden_host))) return set_error(HKHIP_E_BAD_ARGUMENT, "null argument");
    if (!net->partial) return set_error(HKHIP_E_PARTIAL, "hkhip_net_forward_partial needs a partial network");
    if (n == 0) return HKHIP_OK;
    int rc;
    if ((rc = check_loaded(net))) return rc;
    if (hipSetDevice(net->eng->device) != hipSuccess) return set_error(HKHIP_E_DEVICE_FAILED, "hipSetDevice");
    uint32_t max_pos = 0;
    net->last_n = 0;
    net->last_hidden = false;
    if ((rc = stage_items(net, items, n, &max_pos))) return rc;
    const uint64_t bytes = uint64_t(n) * net->cfg.dim * 4;
    NET_TRY(hipMemcpyAsync(net->x, hidden_host, bytes, hipMemcpyHostToDevice, net->eng->cur), "hidden states in");
    if ((rc = forward_staged(net, n, max_pos, false))) return rc;
    NET_TRY(hipMemcpyAsync(hidden_host, net->x, bytes, hipMemcpyDeviceToHost, net->eng->cur), "hidden states out");
    NET_TRY(hipStreamSynchronize(net->eng->cur), "hidden states out");
    net->last_n = n;
    return HKHIP_OK;
}

namespace {
// The logits of rows idx[0..n) of the last pass into net->logits (device), on the engine's stream.
int logits_compute(hkhip_net *net, const uint32_t *idx, uint32_t n);
} // namespace

int hkhip_net_logits_rows(hkhip_net *net, const uint32_t *idx, uint32_t n, float *host_out) {
    if (!net || !idx || !host_out) return set_error(HKHIP_E_BAD_ARGUMENT, "null argument");
    const int rc = logits_compute(net, idx, n);
    if (rc) return rc;
    hipStream_t s = net->eng->cur;
    NET_TRY(hipMemcpyAsync(host_out, net->logits, uint64_t(n) * net->cfg.vocab * 4, hipMemcpyDeviceToHost, s), "logits");
    NET_TRY(hipStreamSynchronize(s), "logits");
    return HKHIP_OK;
}

int hkhip_net_logits_view(hkhip_net *net, const uint32_t *idx, uint32_t n, const float **rows) {
    if (!net || !idx || !rows) return set_error(HKHIP_E_BAD_ARGUMENT, "null argument");
    *rows = nullptr;
    const int rc = logits_compute(net, idx, n);
    if (rc) return rc;
    if (!net->logits_h && hipHostMalloc(reinterpret_cast<void **>(&net->logits_h), uint64_t(net->max_rows) * net->cfg.vocab * 4,
                                        hipHostMallocDefault) != hipSuccess) {
        net->logits_h = nullptr;
        return set_error(HKHIP_E_DEVICE_FAILED, "hipHostMalloc of the pinned logits rows (%u x %u floats)", net->max_rows,
                         net->cfg.vocab);
    }
    hipStream_t s = net->eng->cur;
    NET_TRY(hipMemcpyAsync(net->logits_h, net->logits, uint64_t(n) * net->cfg.vocab * 4, hipMemcpyDeviceToHost, s), "logits");
    NET_TRY(hipStreamSynchronize(s), "logits");
    *rows = net->logits_h;
    return HKHIP_OK;
}

namespace {
int logits_compute(hkhip_net *net, const uint32_t *idx, uint32_t n) {
    if (!net->last_hidden) return set_error(HKHIP_E_BAD_ARGUMENT, "no full forward pass to read logits of");
    if (n < 1 || n > net->max_rows) return set_error(HKHIP_E_BAD_ARGUMENT, "%u rows: 1..%u", n, net->max_rows);
    const hkhip_net_config &c = net->cfg;
    bool run = true;
    for (uint32_t r = 0; r < n; r++) {
        if (idx[r] >= net->last_n) return set_error(HKHIP_E_BAD_ARGUMENT, "row %u: item %u of %u", r, idx[r], net->last_n);
        if (r && idx[r] != idx[r - 1] + 1) run = false;
    }
    if (hipSetDevice(net->eng->device) != hipSuccess) return set_error(HKHIP_E_DEVICE_FAILED, "hipSetDevice");
    hipStream_t s = net->eng->cur;
    const float *src = net->x + uint64_t(idx[0]) * c.dim;
    if (!run) { // gather the rows
        for (uint32_t r = 0; r < n; r++)
            NET_TRY(hipMemcpyAsync(net->lx + uint64_t(r) * c.dim, net->x + uint64_t(idx[r]) * c.dim, uint64_t(c.dim) * 4,
                                   hipMemcpyDeviceToDevice, s), "gather rows");
        src = net->lx;
    }
    // One pass over the output matrix for every requested row (engine.zig:799-817).
    float *const ys[1] = {net->logits};
    return product(net, n, &net->output, 1, src, net->out_norm, ys, nullptr, HKHIP_STORE);
}
} // namespace

void hkhip_net_release(hkhip_net *net, uint64_t seq) {
    if (!net) return;
    for (uint32_t j = 0; j < net->n_slots; j++)
        if (net->used[j] && net->owner[j] == seq) net->used[j] = 0;
}

uint32_t hkhip_net_max_rows(const hkhip_net *net) { return net ? net->max_rows : 0; }
uint32_t hkhip_net_layer_count(const hkhip_net *net) { return net ? net->n_dev : 0; }
int hkhip_net_is_partial(const hkhip_net *net) { return net && net->partial ? 1 : 0; }

int hkhip_net_forward(hkhip_net *net, const uint32_t *tokens, uint32_t n, uint32_t pos0) {
    if (!net || (n && !tokens)) return set_error(HKHIP_E_BAD_ARGUMENT, "null argument");
    std::vector<hkhip_item> items(n);
    for (uint32_t i = 0; i < n; i++) items[i] = hkhip_item{0, tokens[i], pos0 + i};
    if (n && uint64_t(pos0) + n > net->cfg.max_ctx)
        return set_error(HKHIP_E_CONTEXT_FULL, "context full: %u + %u > %u", pos0, n, net->cfg.max_ctx);
    return forward_items(net, items.data(), n, true);
}

int hkhip_net_logits(hkhip_net *net, float *host_out) {
    if (!net || !host_out) return set_error(HKHIP_E_BAD_ARGUMENT, "null argument");
    if (!net->last_hidden) return set_error(HKHIP_E_BAD_ARGUMENT, "no forward pass yet");
    return hkhip_copy_d2h(net->eng, host_out, net->logits, uint64_t(net->cfg.vocab) * 4);
}

const float *hkhip_net_logits_dev(hkhip_net *net) { return net ? net->logits : nullptr; }

uint64_t hkhip_net_layer_bytes(const hkhip_net_config *cfg, const hkhip_net_layer *l) {
    if (!cfg || !l || !config_ok(*cfg)) return 0;
    return layer_dev_bytes(*cfg, *l);
}

uint64_t hkhip_net_bytes_needed(const hkhip_net_config *cfg, const hkhip_net_options *opts, const hkhip_net_layer *layers,
                                hkhip_net_tensor tok_embd, hkhip_net_tensor out_norm, hkhip_net_tensor output) {
    if (!cfg || !layers || !config_ok(*cfg)) return 0;
    const hkhip_net_config &c = *cfg;
    const hkhip_net_options o = opts ? *opts : hkhip_net_options{};
    const uint32_t nl = layer_count(c, o);
    const NetSizes z = net_sizes(c, o.slots ? o.slots : 1, nl, max_rows_of(o), initial_cap(o));
    uint64_t total = z.fixed() + z.per_cap();
    for (uint32_t i = 0; i < nl; i++) {
        const uint64_t lb = layer_dev_bytes(c, layers[i]);
        if (!lb) return 0;
        total += lb;
    }
    if (nl == c.n_layers) {
        if (!block_elems(tok_embd.t) || !block_elems(output.t) || c.dim % block_elems(tok_embd.t) ||
            c.dim % block_elems(output.t))
            return 0;
        (void)out_norm;
        total += weight_layout(tok_embd.t, c.vocab, c.dim).total + uint64_t(c.dim) * 4 +
                 weight_layout(output.t, c.vocab, c.dim).total;
    }
    return total + HKHIP_NET_MARGIN_BYTES;
}

uint64_t hkhip_net_device_bytes(const hkhip_net *net) {
    if (!net) return 0;
    uint64_t total = 0;
    for (const auto &p : net->owned) total += p.second;
    for (const auto &L : net->layers) {
        const hkhip_mat *ms[] = {&L.wqkv, &L.wq, &L.wk, &L.wv, &L.wo, &L.wgu, &L.wd};
        for (const hkhip_mat *m : ms)
            if (m->mem) total += m->dev_bytes;
    }
    if (net->embd.mem) total += net->embd.dev_bytes;
    if (net->output.mem) total += net->output.dev_bytes;
    return total;
}

} // extern "C"
