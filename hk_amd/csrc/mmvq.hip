// Decode matvec (mmvq): the launch side. Kernel design and reference citations: mmvq.hpp.
#include <map>
#include <mutex>
#include <stdlib.h>

#include "mmvq.hpp"

namespace hkhip {

static mv_kernel_t kernel_for(int t, int nt) {
    switch (t) {
    case HKHIP_Q4_K: return pick<HKHIP_Q4_K>(nt);
    case HKHIP_Q6_K: return pick<HKHIP_Q6_K>(nt);
    case HKHIP_Q5_K: return pick<HKHIP_Q5_K>(nt);
    case HKHIP_IQ4_XS: return pick<HKHIP_IQ4_XS>(nt);
    case HKHIP_Q8_0: return pick<HKHIP_Q8_0>(nt);
    case HKHIP_IQ4_NL: return pick<HKHIP_IQ4_NL>(nt);
    case HKHIP_Q4_0: return pick<HKHIP_Q4_0>(nt);
    case HKHIP_Q4_1: return pick<HKHIP_Q4_1>(nt);
    case HKHIP_Q5_0: return pick<HKHIP_Q5_0>(nt);
    case HKHIP_Q5_1: return pick<HKHIP_Q5_1>(nt);
    default: return nullptr;
    }
}

static mv_kernel_t kernelr_for(int t, int nt, int c, int ks, bool norm) {
    switch (t) {
    case HKHIP_Q4_K: return mvr_pick<HKHIP_Q4_K>(nt, c, ks, norm);
    case HKHIP_Q6_K: return mvr_pick<HKHIP_Q6_K>(nt, c, ks, norm);
    case HKHIP_Q5_K: return mvr_pick<HKHIP_Q5_K>(nt, c, ks, norm);
    case HKHIP_IQ4_XS: return mvr_pick<HKHIP_IQ4_XS>(nt, c, ks, norm);
    case HKHIP_Q8_0: return mvr_pick<HKHIP_Q8_0>(nt, c, ks, norm);
    case HKHIP_IQ4_NL: return mvr_pick<HKHIP_IQ4_NL>(nt, c, ks, norm);
    case HKHIP_Q4_0: return mvr_pick<HKHIP_Q4_0>(nt, c, ks, norm);
    case HKHIP_Q4_1: return mvr_pick<HKHIP_Q4_1>(nt, c, ks, norm);
    case HKHIP_Q5_0: return mvr_pick<HKHIP_Q5_0>(nt, c, ks, norm);
    case HKHIP_Q5_1: return mvr_pick<HKHIP_Q5_1>(nt, c, ks, norm);
    default: return nullptr;
    }
}

static mv_kernel_t kernels_for(int t, int lg, int nw) {
    switch (t) {
    case HKHIP_Q4_K: return mvs_pick<HKHIP_Q4_K>(lg, nw);
    case HKHIP_Q6_K: return mvs_pick<HKHIP_Q6_K>(lg, nw);
    case HKHIP_Q5_K: return mvs_pick<HKHIP_Q5_K>(lg, nw);
    case HKHIP_IQ4_XS: return mvs_pick<HKHIP_IQ4_XS>(lg, nw);
    case HKHIP_Q8_0: return mvs_pick<HKHIP_Q8_0>(lg, nw);
    case HKHIP_IQ4_NL: return mvs_pick<HKHIP_IQ4_NL>(lg, nw);
    case HKHIP_Q4_0: return mvs_pick<HKHIP_Q4_0>(lg, nw);
    case HKHIP_Q4_1: return mvs_pick<HKHIP_Q4_1>(lg, nw);
    case HKHIP_Q5_0: return mvs_pick<HKHIP_Q5_0>(lg, nw);
    case HKHIP_Q5_1: return mvs_pick<HKHIP_Q5_1>(lg, nw);
    default: return nullptr;
    }
}

// Short one-token launches: at most this many work units in all (measured on MI355X: the Qwen3-0.6B
// products, 49K-98K units, gain 0.2-0.5 us each; the Llama-3-8B q/k/v and o, 262K-393K, lose as
// much).
constexpr uint64_t MVS_MAX_UNITS = 131072;
// Short one-token launches: workgroups aimed for (0: none), waves per workgroup, and how many
// steps of lanes per row above the packing the row length allows.
struct MvsPolicy {
    uint32_t wgs;
    int nw, lg_up;
};
static MvsPolicy mvs_policy() {
    MvsPolicy p{512, 4, 0};
#ifdef HKHIP_MV_SWEEP
    if (const char *e = getenv("HKHIP_MV_SMALL_WGS")) p.wgs = uint32_t(atoi(e));
    if (const char *e = getenv("HKHIP_MVS_NW")) p.nw = atoi(e);
    if (const char *e = getenv("HKHIP_MVS_LGUP")) p.lg_up = atoi(e);
#endif
    return p;
}

// Resident workgroups per CU for a kernel at an LDS size (cached; the first call per kernel also
// raises its dynamic-LDS limit to the full 160 KB).
static int resident_per_cu(mv_kernel_t k, int threads, uint32_t lds) {
    static std::mutex mu;
    static std::map<std::pair<void *, uint32_t>, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto key = std::make_pair(reinterpret_cast<void *>(k), lds);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                              int(MV_LDS_MAX));
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, threads, lds) != hipSuccess || n < 1) n = 1;
    cache[key] = n;
    return n;
}

static int cu_count() {
    static int n = 0;
    if (!n) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
    }
    return n;
}


// Where a launch finds its input: an f32 array, or the planes of a prepared activation buffer.
struct MvAct {
    const float *x;
    const int8_t *qs;
    const float *d;
    const int16_t *bs;
};

// The input of tokens t0.. of `a`.
static MvAct mv_act_at(const MvAct &a, bool kq, uint32_t K, uint32_t t0) {
    MvAct r{};
    if (a.x) {
        r.x = a.x + uint64_t(t0) * K;
    } else {
        r.qs = a.qs + uint64_t(t0) * K;
        r.d = a.d + uint64_t(t0) * (K / (kq ? 256 : 32));
        r.bs = a.bs + uint64_t(t0) * (K / 16);
    }
    return r;
}

// One launch (register kernel) or a few (LDS kernel) for at most 8 tokens.
static hipError_t launch_mv_chunk(int t, const MvPartDesc *parts, int nparts, uint32_t K, const MvAct &act,
                                  uint32_t n, int mode, const float *norm, float eps, hipStream_t s) {
    const float *x = act.x;
    if (n < 1 || n > 8 || nparts < 1 || nparts > MV_PARTS) return hipErrorInvalidValue;
    const bool kq = act_kind(t) == HKHIP_ACT_Q8K;
    {
        // Register kernel when the shape fits it.
        const uint32_t units = kq ? K / 64 : K / 32;
        const int nt = n == 1 ? 1 : n == 2 ? 2 : n <= 4 ? 4 : 8;
        int c = 1, ks = 1;
        while (c < 8 && 64u * c < units) c *= 2;
        if (64u * c < units || c > mvr_cmax(t, nt)) {
            // Rows too long for one wave's registers: slices of cmax units per lane.
            c = mvr_cmax(t, nt);
            while (ks < 8 && 64u * c * ks < units) ks *= 2;
        }
        mv_kernel_t k = 64u * c * ks >= units ? kernelr_for(t, nt, c, ks, norm != nullptr) : nullptr;
        uint32_t total_rows = 0;
        for (int i = 0; i < nparts; i++) total_rows += parts[i].rows;
        // One token, rows of at most 64 units. Rows of up to 32 units are packed 2^lg lanes per
        // row (lg 4 or 5) instead of leaving lanes idle. Short launches (up to 16384 rows) run
        // small workgroups with few rows per wave, so that every wave issues all its loads at once
        // and the launch spreads over the CUs: a launch of a few MB is latency-bound.
        int lg = 6, snw = 0;
        uint32_t spw = 0; // row steps per wave of a short launch
        if (k && nt == 1 && ks == 1 && c == 1) {
            lg = units <= 16 ? 4 : units <= 32 ? 5 : 6;
            const MvsPolicy P = mvs_policy();
            if (P.wgs && uint64_t(total_rows) * units <= MVS_MAX_UNITS) {
                snw = P.nw;
                lg = lg + P.lg_up > 6 ? 6 : lg + P.lg_up;
                const uint32_t rs = 64u >> lg, per = rs * uint32_t(snw) * P.wgs;
                spw = (total_rows + per - 1) / per;
                k = kernels_for(t, lg, snw);
            } else if (lg < 6) {
                k = kernels_for(t, lg, 8);
            }
        }
        // A fused RMS norm needs LDS for one partial sum per 16 inputs after the staging area.
        const uint32_t nflat = (nt == 1 ? 1u : n) * K;
        const uint32_t norm_bytes = norm ? nflat / 4 + 64 : 0; // partial sums, then the tokens' factors
        if (norm && !x) return hipErrorNotSupported;
        if (k && x) {
            // An f32 input is staged whole in LDS; when it does not fit, the LDS kernel splits the
            // tokens over launches.
            uint32_t need = mvr_lds_bytes(int(n), K, kq);
            if (ks > 1) need = ((need + 15) & ~15u) + uint32_t(mvr_nw(t, nt, c)) * 64 * nt * 4;
            if (norm) need = ((need + 15) & ~15u) + norm_bytes;
            if (need > MV_LDS_MAX) k = nullptr;
        }
        if (!k && norm) return hipErrorNotSupported;
        if (k) {
            MvArgs a{};
            uint32_t rows = 0;
            for (int i = 0; i < nparts; i++) {
                const WLayout W = weight_layout(t, parts[i].rows, K);
                a.p[i].w = parts[i].w;
                a.p[i].ws = reinterpret_cast<const uint16_t *>(parts[i].w + W.scale_off);
                a.p[i].y = parts[i].y;
                a.p[i].bias = parts[i].bias;
                a.p[i].rows = parts[i].rows;
                a.p[i].gstart = rows;
                rows += parts[i].rows;
            }
            for (int i = nparts; i < MV_PARTS; i++) a.p[i].gstart = 0xffffffffu;
            a.nparts = uint32_t(nparts);
            a.ngroups = rows;
            a.K = K;
            a.mode = mode;
            a.ntok = n;
            a.x = act.x;
            a.gqs = act.qs;
            a.gd = act.d;
            a.gbs = act.bs;
            a.norm = norm;
            a.eps = eps;
            if (rows == 0) return hipSuccess;
            // Rows dealt in turn (measured on the Llama-3-8B decode step: 1.234 -> 1.191 ms; the
            // fused gate/up 14.0 -> 13.4 us); the kernel keeps contiguous ranges where that cannot
            // apply.
            a.interleave = 1;
            if (spw) {
                const uint32_t rs = 64u >> lg;
                const uint32_t lds = x ? (norm ? mvr_norm_offset(1, K, kq, 0) + norm_bytes : mvr_lds_bytes(1, K, kq)) : 0;
                if (lds > MV_LDS_MAX) return hipErrorInvalidValue;
                const uint32_t waves = (rows + rs * spw - 1) / (rs * spw);
                hipLaunchKernelGGL(k, dim3((waves + snw - 1) / snw), dim3(snw * 64), lds, s, a);
                return hipGetLastError();
            }
            const int R = mvr_rows(nt, c) << (6 - lg); // rows per wave step (packed: R slots of 64 >> lg)
            const int nw = mvr_nw(t, nt, c), nrg = nw / ks;
            uint32_t lds = x ? mvr_lds_bytes(int(n), K, kq) : 0;
            if (ks > 1) lds = ((lds + 15) & ~15u) + uint32_t(nw) * 64 * nt * 4; // partials
            if (norm) lds = mvr_norm_offset(nt == 1 ? 1u : n, K, kq, ks > 1 ? uint32_t(nw) * 64 * nt * 4 : 0) + norm_bytes;
            if (lds > MV_LDS_MAX) return hipErrorInvalidValue;
            const uint32_t cap = uint32_t(cu_count() * resident_per_cu(k, nw * 64, lds));
            const uint32_t want = (rows + nrg * R - 1) / (nrg * R);
            uint32_t grid = want < cap ? want : cap;
            // One token and up to 16384 rows: one workgroup per CU streams longer row ranges and
            // stages the input fewer times (measured at 14336x4096: Q4_K 10.1 -> 9.0 us, IQ4_NL
            // 11.5 -> 10.3 us; 6144x4096 6.6 -> 5.8 us); larger launches keep more bytes in
            // flight with more workgroups.
            if (nt == 1 && rows <= 16384 && grid > uint32_t(cu_count())) grid = uint32_t(cu_count());
            // At most 64 rows per row group (each lane keeps one row's result); extra workgroups
            // queue.
            const uint32_t need = (rows + 64u * nrg - 1) / (64u * nrg);
            if (grid < need) grid = need;
            hipLaunchKernelGGL(k, dim3(grid), dim3(nw * 64), lds, s, a);
            return hipGetLastError();
        }
    }
    if (norm) return hipErrorNotSupported;
    // Tokens per launch: as many as the LDS holds (all 8 at every BASELINE shape).
    int per = int(n);
    while (per > 1 && mv_lds_bytes(per, K, kq) > MV_LDS_MAX) per--;
    if (mv_lds_bytes(per, K, kq) > MV_LDS_MAX) return hipErrorInvalidValue;
    const uint32_t units = kq ? K / 64 : K / 32;
    // Lanes per row: enough that a row takes one step of UNR units per lane when it can.
    const uint32_t unr = MV_UNR;
    const uint32_t want_lanes = (units + unr - 1) / unr;
    int lg = 0;
    while ((1u << lg) < want_lanes && lg < 6) lg++;
    if (mode == HKHIP_SILU_MUL && lg > 5) lg = 5; // a gate/up pair within one wave
    const uint32_t rpw = 64u >> lg;
    const int nw = MV_NW;
    for (uint32_t t0 = 0; t0 < n; t0 += per) {
        const int nt = int(n - t0 < uint32_t(per) ? n - t0 : uint32_t(per));
        MvArgs a{};
        uint32_t groups = 0;
        for (int i = 0; i < nparts; i++) {
            const WLayout W = weight_layout(t, parts[i].rows, K);
            a.p[i].w = parts[i].w;
            a.p[i].ws = reinterpret_cast<const uint16_t *>(parts[i].w + W.scale_off);
            a.p[i].y = parts[i].y + uint64_t(t0) * (mode == HKHIP_SILU_MUL ? parts[i].rows / 2 : parts[i].rows);
            a.p[i].bias = parts[i].bias;
            a.p[i].rows = parts[i].rows;
            a.p[i].gstart = groups;
            groups += (parts[i].rows + rpw - 1) / rpw;
        }
        for (int i = nparts; i < MV_PARTS; i++) a.p[i].gstart = 0xffffffffu;
        a.nparts = uint32_t(nparts);
        a.ngroups = groups;
        a.K = K;
        a.mode = mode;
        a.lpr_log2 = lg;
        const MvAct at = mv_act_at(act, kq, K, t0);
        a.x = at.x;
        a.gqs = at.qs;
        a.gd = at.d;
        a.gbs = at.bs;
        if (groups == 0) continue;
        mv_kernel_t k = kernel_for(t, nt);
        if (!k) return hipErrorInvalidValue;
        const uint32_t lds = mv_lds_bytes(nt, K, kq);
        // Enough workgroups for every row group, and at least one per CU while there are row
        // groups to give them (small matrices still spread their bytes over every CU).
        const uint32_t ncu = uint32_t(cu_count());
        uint32_t want = (groups + nw - 1) / nw;
        if (want < ncu) want = groups < ncu ? groups : ncu;
        const uint32_t cap = uint32_t(cu_count() * resident_per_cu(k, nw * 64, lds));
        const uint32_t grid = want < cap ? want : cap;
        hipLaunchKernelGGL(k, dim3(grid), dim3(nw * 64), lds, s, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_mmvq_parts(int t, const MvPartDesc *parts, int nparts, uint32_t K, const float *x,
                             const uint8_t *xq, uint32_t n, int mode, hipStream_t s) {
    return launch_mmvq_parts_norm(t, parts, nparts, K, x, xq, n, mode, nullptr, 0.0f, s);
}

hipError_t launch_mmvq_parts_norm(int t, const MvPartDesc *parts, int nparts, uint32_t K, const float *x,
                                  const uint8_t *xq, uint32_t n, int mode, const float *norm, float eps,
                                  hipStream_t s) {
    if (n < 1 || nparts < 1 || nparts > MV_PARTS) return hipErrorInvalidValue;
    if (norm && !x) return hipErrorNotSupported;
    if (fallback_type(t)) return norm ? hipErrorNotSupported : launch_fb_mv(t, parts, nparts, K, x, xq, n, mode, s);
    const bool kq = act_kind(t) == HKHIP_ACT_Q8K;
    // Q4_K and Q6_K from 4 tokens with a prepared input: the small-batch MFMA kernel (it needs the
    // quantizer's token-interleaved planes, so not for an f32 input).
    if (!x && n >= SK_MIN_TOKENS) {
        bool sk = true;
        for (int i = 0; i < nparts; i++) sk = sk && mmsk_supports(t, parts[i].rows, K, n);
        if (sk) return launch_mmsk_parts(t, parts, nparts, K, xq, n, mode, s);
    }
    MvAct act{};
    if (x) {
        act.x = x;
    } else {
        const ActLayout A = act_layout(n, K);
        act.qs = reinterpret_cast<const int8_t *>(xq + (kq ? A.k_qs : A.a8_qs));
        act.d = reinterpret_cast<const float *>(xq + (kq ? A.k_d : A.a8_d));
        act.bs = reinterpret_cast<const int16_t *>(xq + A.k_bs);
    }
    // Up to 8 tokens per launch; more run as consecutive chunks of 8.
    for (uint32_t t0 = 0; t0 < n; t0 += 8) {
        const uint32_t nc = n - t0 < 8 ? n - t0 : 8;
        MvPartDesc pc[MV_PARTS];
        for (int i = 0; i < nparts; i++) {
            pc[i] = parts[i];
            pc[i].y = parts[i].y + uint64_t(t0) * (mode == HKHIP_SILU_MUL ? parts[i].rows / 2 : parts[i].rows);
        }
        const hipError_t e = launch_mv_chunk(t, pc, nparts, K, t0 ? mv_act_at(act, kq, K, t0) : act, nc, mode, norm, eps, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_mmvq(int t, const uint8_t *w, uint32_t rows, uint32_t cols, const uint8_t *xq, uint32_t n,
                       float *y, const float *bias, int mode, hipStream_t s) {
    MvPartDesc p{w, y, bias, rows};
    return launch_mmvq_parts(t, &p, 1, cols, nullptr, xq, n, mode, s);
}

} // namespace hkhip
