// k_moe.hip - MUL_MAT_ID routing, the MoE router (softmax / top-k) and the
// combine of the experts' outputs on gfx950.
//
// Role of the reference's kernel_moe_route_tiles (P01:2417-2444): route
// work-groups count the (token, slot) pairs of every expert in LDS, scan the
// counts and scatter the pairs into per-expert tasks of up to kMaxTaskCols
// activation columns (each work-group its own slice of the pairs), which the
// GEMV kernel then runs as "few columns against one expert": every touched
// expert's weights are streamed once per task.
// The expert counts are scanned in parallel (a wave scan by shuffles, then the
// 16 wave totals): a serial scan by one thread over 512 experts took 24 us.
// Pair (slot i, token t) reads activation column (i % ne11) + t * ne11 and
// writes dst + t * nb2 + i * nb1 (P01:3916-3922).  A negative id writes a zero
// row (the reference's expert-cache rule, P02:98-103); an id at or past n_as,
// which ggml-cpu asserts on (P02:105), also writes a zero row - nothing reads
// outside the stack - and sets the context's error flag, which
// qmm_synchronize reports.  Such pairs go to one more bucket whose tasks
// (mat = -1) the GEMV turns into zero rows, so the route writes no dst and one
// route serves every product that shares the ids.
#include "qmm_device.h"

#include <algorithm>
#include <cstdlib>

namespace qmm {
namespace {

constexpr int kRouteThreads = 1024;
constexpr int kHeld = 16;               // pairs a route thread keeps in registers (16384 in all)

// Work-group rw of nrw route work-groups (kRouteThreads each); sm = [2 nbk] ints of LDS, s_wsum =
// [kRouteThreads / 64]; tasks of up to TC pairs (GEMV tasks: 8, the grouped GEMM's units: 64).
// The pairs are cut into nrw contiguous slices and each work-group scatters its own: one
// work-group's scattered 16-byte task stores took 4.3 of the 10.8 us at 10240 pairs.  Every
// work-group counts every pair (the ids are read again, from L2), so each knows the buckets'
// totals, hence the same task layout, and how many pairs of each bucket the slices ahead of its
// own hold, hence where its pairs go: no work-group waits for another.
template <int TC>
__device__ __forceinline__ void route_body(const RouteArgs & r, TaskOf<TC> * __restrict__ tasks,
                                           int32_t * __restrict__ ntasks, int32_t * sm, int32_t * s_wsum, uint32_t nrw,
                                           uint32_t rw) {
    const int64_t nbk = r.n_as + 1 + r.shared;   // buckets: the experts, [the shared expert,] the invalid ids
    const int32_t inv = (int32_t)(r.n_as + r.shared);
    int32_t * before = sm;              // [nbk] pairs of the earlier slices, later this slice's fill cursor
    int32_t * total = sm + nbk;         // [nbk] pairs in all, later the bucket's first task
    const int tid = threadIdx.x;
    // pair p = t nu + i in 32 bits (the launcher keeps the pair count below 2^31)
    const uint32_t nu = (uint32_t)(r.n_used + r.shared), n11 = (uint32_t)r.ne11;
    const uint32_t npairs = nu * (uint32_t)r.T;
    const uint32_t per = (npairs + nrw - 1) / nrw;
    const uint32_t lo = std::min(npairs, rw * per), hi = std::min(npairs, lo + per);   // this slice
    constexpr int32_t kSharedId = -2147483647 - 1;                // (slot n_used with the shared expert: no id)
    auto id_at = [&](uint32_t t, uint32_t i) {
        if (r.shared && i == (uint32_t)r.n_used) return kSharedId;
        return *reinterpret_cast<const int32_t *>(reinterpret_cast<const char *>(r.ids) + (size_t)t * r.ids_nb1 +
                                                  (size_t)i * r.ids_nb0);
    };
    auto bucket = [&](int32_t e) {
        if (e == kSharedId) return (int32_t)r.n_as;
        if (e >= r.n_as) *r.bad_id = 1;
        return (e >= 0 && e < r.n_as) ? e : inv;
    };
    // pairs p, p + kRouteThreads, ...: (t, i) by steps (t by dq and i by dr; one division per
    // run of pairs instead of one per pair)
    const uint32_t dq = (uint32_t)kRouteThreads / nu, dr = (uint32_t)kRouteThreads - dq * nu;
    auto step = [&](uint32_t & t, uint32_t & i) {
        i += dr;
        t += dq;
        if (i >= nu) {
            i -= nu;
            ++t;
        }
    };
    // count the pairs of [b, e) into c, kHeld per thread at a time (every id of a run requested
    // before any is used: one memory round trip per run, not one per pair)
    auto count = [&](uint32_t b, uint32_t e, int32_t * c) {
        for (uint32_t p0 = b + (uint32_t)tid; p0 < e; p0 += (uint32_t)kHeld * kRouteThreads) {
            uint32_t t = p0 / nu, i = p0 - t * nu;
            int32_t v[kHeld];
#pragma unroll
            for (int j = 0; j < kHeld; ++j) {
                v[j] = p0 + (uint32_t)j * kRouteThreads < e ? id_at(t, i) : 0;
                step(t, i);
            }
#pragma unroll
            for (int j = 0; j < kHeld; ++j)
                if (p0 + (uint32_t)j * kRouteThreads < e) atomicAdd(&c[bucket(v[j])], 1);
        }
    };
    // the thread's pairs p = tid + j kRouteThreads (j < kHeld, every pair up to kHeld
    // kRouteThreads): all their ids requested at once (one memory round trip), their buckets kept
    // in registers for both counts and the scatter; pairs past them take more runs (count)
    constexpr uint32_t kHeldPairs = (uint32_t)kHeld * kRouteThreads;
    int32_t held[kHeld];
    const uint32_t t0 = (uint32_t)tid / nu, i0 = (uint32_t)tid - t0 * nu;
    {
        uint32_t t = t0, i = i0;
#pragma unroll
        for (int j = 0; j < kHeld; ++j) {
            held[j] = (uint32_t)tid + (uint32_t)j * kRouteThreads < npairs ? id_at(t, i) : 0;
            step(t, i);
        }
    }
    for (int64_t e = tid; e < nbk; e += kRouteThreads) before[e] = total[e] = 0;
    __syncthreads();
    // total: every pair; before: the pairs of the slices ahead of this one (one pass: counting
    // before first and copying it into total cost two more barriers, slower at every size)
#pragma unroll
    for (int j = 0; j < kHeld; ++j) {
        const uint32_t p = (uint32_t)tid + (uint32_t)j * kRouteThreads;
        if (p < npairs) {
            held[j] = bucket(held[j]);
            atomicAdd(&total[held[j]], 1);
            if (p < lo) atomicAdd(&before[held[j]], 1);
        }
    }
    count(kHeldPairs, lo, before);
    count(kHeldPairs, npairs, total);
    __syncthreads();
    // exclusive scan of the buckets' task counts, in place (total becomes the first task): thread
    // tid owns buckets [tid per, tid per + per), a wave scan by shuffles, then the 16 wave totals
    // through LDS; the owner of bucket e writes its task headers in work-group e % nrw (the
    // invalid bucket's tasks: mat = -1, zero rows)
    {
        const int64_t bper = (nbk + kRouteThreads - 1) / kRouteThreads, e0 = tid * bper;
        int32_t local = 0;
        for (int64_t k = 0; k < bper; ++k)
            if (e0 + k < nbk) local += (total[e0 + k] + TC - 1) / TC;
        const int lane = tid & 63, wave = tid >> 6;
        int32_t x = local;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int32_t v = __shfl_up(x, d, 64);
            if (lane >= d) x += v;
        }
        int32_t excl;
        if (nbk <= 64) {                                          // uniform
            // every bucket in wave 0 (one a thread): its scan is the whole scan, no cross-wave
            // step (two barriers and a serial pass over the 16 wave sums: ~1 of the 1.36 us this
            // phase took at 16 experts)
            excl = x - local;
            if (tid == 63 && rw == 0) *ntasks = x;
        } else {
            if (lane == 63) s_wsum[wave] = x;
            __syncthreads();
            if (tid == 0) {
                int32_t acc = 0;
                for (int w = 0; w < kRouteThreads / 64; ++w) {
                    const int32_t t = s_wsum[w];
                    s_wsum[w] = acc;
                    acc += t;
                }
                if (rw == 0) *ntasks = acc;
            }
            __syncthreads();
            excl = x - local + s_wsum[wave];
        }
        for (int64_t k = 0; k < bper; ++k) {
            const int64_t e = e0 + k;
            if (e >= nbk) break;
            const int32_t c = total[e], nt = (c + TC - 1) / TC;
            total[e] = excl;
            if ((uint32_t)(e % nrw) == rw)
                for (int32_t q = 0; q < nt; ++q) {
                    TaskOf<TC> & T = tasks[excl + q];
                    T.mat = e < r.n_as ? (int32_t)(QMM_RED == 7 ? (e + 1) % r.n_as : e) : e < inv ? (int32_t)e : -1;   // (mutation 7: next expert)
                    T.ncols = (c - q * TC) < TC ? (c - q * TC) : TC;
                }
            excl += nt;
        }
    }
    __syncthreads();
    // the task slot of pair (t, i) of bucket b: its column and dst offset (one 16-byte store)
    auto place = [&](uint32_t t, uint32_t i, int32_t b) {
        const int64_t q = (int64_t)total[b] * TC + atomicAdd(&before[b], 1);
        TaskCol c;
        c.col = b != inv ? (int32_t)((n11 == nu ? i : i % n11) + t * n11) : 0;
        c.pad = 0;
        c.dst_off = (int64_t)t * r.dst_nb2 + (int64_t)i * r.dst_nb1;
        tasks[q / TC].c[q % TC] = c;
    };
    {
        uint32_t t = t0, i = i0;
#pragma unroll
        for (int j = 0; j < kHeld; ++j) {
            const uint32_t p = (uint32_t)tid + (uint32_t)j * kRouteThreads;
            if (p >= lo && p < hi) place(t, i, held[j]);
            step(t, i);
        }
    }
    for (uint32_t p = std::max(lo, kHeldPairs) + (uint32_t)tid; p < hi; p += kRouteThreads) {   // (pairs past the held)
        const uint32_t t = p / nu, i = p - t * nu;
        place(t, i, bucket(id_at(t, i)));
    }
}

template <int TC>
__global__ __launch_bounds__(kRouteThreads) void k_route(RouteArgs r, TaskOf<TC> * __restrict__ tasks,
                                                         int32_t * __restrict__ ntasks) {
    extern __shared__ int32_t sm[];
    __shared__ int32_t s_wsum[kRouteThreads / 64];
    route_body<TC>(r, tasks, ntasks, sm, s_wsum, gridDim.x, blockIdx.x);
}

// MUL_MAT_ID's two independent preparations in one launch: work-groups [0, nrw) route, the
// others quantize the activations (the q8_0 or q8_K pass of the quantization launch, no dst
// zeroing).  At decode both are a few microseconds of latency each; side by side the GEMV
// waits for the longer one instead of their sum.
template <int VDT, int TC>
__global__ __launch_bounds__(kRouteThreads) void k_quant_route(F32Cols src, int64_t K, int64_t ncols, ActBuf a,
                                                               RouteArgs r, uint32_t nrw, TaskOf<TC> * __restrict__ tasks,
                                                               int32_t * __restrict__ ntasks) {
    extern __shared__ int32_t sm[];
    __shared__ int32_t s_wsum[kRouteThreads / 64];
    if (blockIdx.x < nrw) {                                       // uniform
        route_body<TC>(r, tasks, ntasks, sm, s_wsum, nrw, blockIdx.x);
        return;
    }
    const int64_t t = (int64_t)(blockIdx.x - nrw) * kRouteThreads + threadIdx.x;
    if (VDT == QMM_TYPE_Q8_0) quant_q8_0_at(src, K, ncols, a, t);
    else quant_q8_K_at(src, K, ncols, a, t);
}

// ---- the router: softmax -> top-k -> normalized weights ------------------------------------
// One wave per token (a one-wave work-group) runs topk_wave (qmm_device.h: the role of the
// reference's fused router, P09:899-1000); the fused MoE FFN's gate/up launch runs the same
// function in each work-group's first wave.
constexpr int kTopkMaxExperts = 1024;

template <int NPER>
__global__ __launch_bounds__(64) void k_topk(TopkArgs a) {
    __shared__ uint32_t cand_key[kTopkMaxExperts];
    __shared__ int cand_exp[kTopkMaxExperts];
    __shared__ float ranked_p[32];
    const int64_t t = blockIdx.x;
    topk_wave<NPER>(reinterpret_cast<const float *>(a.logits + t * a.nbl1), a.n_expert, a.k, a.cmin, a.cmax,
                    (int)threadIdx.x, cand_key, cand_exp, ranked_p, reinterpret_cast<int32_t *>(a.ids + t * a.nbi1),
                    reinterpret_cast<float *>(a.w + t * a.nbw1));
}

// ---- the combine: dst[:, t] = sum_j w[j, t] experts[:, j, t] (+ shared[:, t] sigmoid(g[t]))
// in llama.cpp's order: the products rounded, added slot by slot, then the gated shared
// expert added (contraction off: ggml-cpu's MUL then ADDs round every product).
// grid (ceil(M / 256), tokens from t0): the position without a division
__global__ __launch_bounds__(256) void k_combine(CombineArgs a, int64_t t0) {
#pragma clang fp contract(off)
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x, t = t0 + blockIdx.y;
    if (m >= a.M) return;
    const char * e = a.experts + t * a.enb2 + m * 4;
    const float * w = reinterpret_cast<const float *>(a.w + t * a.wnb1);
    float y = reinterpret_cast<const float *>(e)[0] * w[0];
    for (int j = 1; j < a.k; ++j) y = y + *reinterpret_cast<const float *>(e + j * a.enb1) * w[j];
    if (a.shared) {                                               // (no gate logit: the shared row unweighted)
        float sg = 1.0f;
        if (a.gate) sg = 1.0f / (1.0f + expf(-*reinterpret_cast<const float *>(a.gate + t * a.gnb1)));
        y = y + (a.gate ? *reinterpret_cast<const float *>(a.shared + t * a.snb1 + m * 4) * sg
                        : *reinterpret_cast<const float *>(a.shared + t * a.snb1 + m * 4));
    }
    *reinterpret_cast<float *>(a.dst + t * a.dnb1 + m * 4) = y;
}

}  // namespace

hipError_t launch_topk(const TopkArgs & a, hipStream_t s) {
    if (a.n_expert < 1 || a.n_expert > 1024 || a.k < 1 || a.k > 32 || a.k > a.n_expert || a.n_tok < 1) return hipErrorInvalidValue;
    if (a.n_tok > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 g((unsigned)a.n_tok), b(64);                       // one wave per token
    const int nper = (a.n_expert + 63) / 64;
    if (nper <= 1) k_topk<1><<<g, b, 0, s>>>(a);
    else if (nper <= 2) k_topk<2><<<g, b, 0, s>>>(a);
    else if (nper <= 4) k_topk<4><<<g, b, 0, s>>>(a);
    else if (nper <= 8) k_topk<8><<<g, b, 0, s>>>(a);
    else k_topk<16><<<g, b, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_combine(const CombineArgs & a, hipStream_t s) {
    if (a.M < 1 || a.T < 1 || a.k < 1 || a.M * a.T >= ((int64_t)1 << 40) || (a.M + 255) / 256 > 0x7fffffff)
        return hipErrorInvalidValue;
    for (int64_t t0 = 0; t0 < a.T; t0 += 65535) {              // (grid y: at most 65535 tokens a launch)
        k_combine<<<dim3((unsigned)((a.M + 255) / 256), (unsigned)std::min<int64_t>(65535, a.T - t0)), 256, 0, s>>>(a, t0);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

namespace {
// route work-groups: one per kRouteWgPairs pairs, at most kRouteMaxWg (QMM_ROUTE_WG overrides:
// a count, for tuning); each one counts every pair and scatters its slice
constexpr int64_t kRouteWgPairs = 1024;
constexpr int64_t kRouteMaxWg = 8;
uint32_t route_wgs(int64_t npairs) {
    static const int64_t env = [] {
        const char * e = getenv("QMM_ROUTE_WG");
        return e ? std::max<int64_t>(1, std::min<int64_t>(64, atoll(e))) : 0;
    }();
    const int64_t n = env ? env : std::min(kRouteMaxWg, (npairs + kRouteWgPairs - 1) / kRouteWgPairs);
    return (uint32_t)std::max<int64_t>(1, n);
}

bool route_ok(const RouteArgs & r, size_t * lds) {
    *lds = (size_t)(r.n_as + 1 + r.shared) * 2 * sizeof(int32_t);
    return *lds <= 64 * 1024 && (r.n_used + r.shared) * r.T < ((int64_t)1 << 31) && r.shared >= 0 && r.shared <= 1 &&
           r.n_used >= 1 && r.T >= 1;
}

template <int TC>
hipError_t route_t(const RouteArgs & r, TaskOf<TC> * tasks, int32_t * ntasks, hipStream_t s) {
    size_t lds;
    if (!route_ok(r, &lds)) return hipErrorInvalidValue;
    k_route<TC><<<route_wgs((r.n_used + r.shared) * r.T), kRouteThreads, lds, s>>>(r, tasks, ntasks);
    return hipGetLastError();
}

template <int TC>
hipError_t quant_route_t(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, const RouteArgs & r,
                         TaskOf<TC> * tasks, int32_t * ntasks, hipStream_t s) {
    size_t lds;
    if (!route_ok(r, &lds) || K <= 0 || ncols < 0 || a.ldk % 256 || a.ldk < K) return hipErrorInvalidValue;
    const uint32_t nrw = route_wgs((r.n_used + r.shared) * r.T);
    const int64_t nq = a.vdt == QMM_TYPE_Q8_0 ? ncols * (a.ldk / 4) : ncols * (a.ldk / 256) * 64;
    const int64_t grid = nrw + (nq + kRouteThreads - 1) / kRouteThreads;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    if (a.vdt == QMM_TYPE_Q8_0)
        k_quant_route<QMM_TYPE_Q8_0, TC><<<dim3((unsigned)grid), kRouteThreads, lds, s>>>(src, K, ncols, a, r, nrw, tasks,
                                                                                          ntasks);
    else
        k_quant_route<QMM_TYPE_Q8_K, TC><<<dim3((unsigned)grid), kRouteThreads, lds, s>>>(src, K, ncols, a, r, nrw, tasks,
                                                                                          ntasks);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_route(const RouteArgs & r, int32_t *, GemvTask * tasks, int32_t * ntasks, hipStream_t s) {
    return route_t(r, tasks, ntasks, s);
}
hipError_t launch_route(const RouteArgs & r, int32_t *, GemmUnit * units, int32_t * nunits, hipStream_t s) {
    return route_t(r, units, nunits, s);
}
hipError_t launch_quant_route(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, const RouteArgs & r,
                              int32_t *, GemvTask * tasks, int32_t * ntasks, hipStream_t s) {
    return quant_route_t(src, K, ncols, a, r, tasks, ntasks, s);
}
hipError_t launch_quant_route(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, const RouteArgs & r,
                              int32_t *, GemmUnit * units, int32_t * nunits, hipStream_t s) {
    return quant_route_t(src, K, ncols, a, r, units, nunits, s);
}

}  // namespace qmm
