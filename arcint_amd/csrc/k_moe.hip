// k_moe.hip - MUL_MAT_ID routing, the MoE router (softmax / top-k) and the
// combine of the experts' outputs on gfx950.
//
// Role of the reference's kernel_moe_route_tiles (P01:2417-2444): one
// work-group counts the (token, slot) pairs of every expert in LDS, scans the
// counts and scatters the pairs into per-expert tasks of up to kMaxTaskCols
// activation columns, which the GEMV kernel then runs as "few columns against
// one expert": every touched expert's weights are streamed once per task.
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

namespace qmm {
namespace {

constexpr int kRouteThreads = 1024;

// one work-group of kRouteThreads; sm = [2 (n_as + 1)] ints of LDS, s_wsum = [kRouteThreads / 64];
// tasks of up to TC pairs (GEMV tasks: 8, the grouped GEMM's units: 64)
template <int TC>
__device__ __forceinline__ void route_body(const RouteArgs & r, int32_t * __restrict__ scratch,
                                           TaskOf<TC> * __restrict__ tasks, int32_t * __restrict__ ntasks,
                                           int32_t * sm, int32_t * s_wsum) {
    const int64_t nbk = r.n_as + 1;     // buckets: the experts, then the invalid ids
    int32_t * cnt = sm;                 // [nbk] pair count, later the fill cursor
    int32_t * tstart = sm + nbk;        // [nbk] first task of each bucket
    const int tid = threadIdx.x;
    const int64_t npairs = r.n_used * r.T;
    for (int64_t e = tid; e < nbk; e += kRouteThreads) cnt[e] = 0;
    __syncthreads();
    for (int64_t p = tid; p < npairs; p += kRouteThreads) {
        const int64_t t = p / r.n_used, i = p % r.n_used;
        const int32_t e = *reinterpret_cast<const int32_t *>(reinterpret_cast<const char *>(r.ids) + t * r.ids_nb1 + i * r.ids_nb0);
        const int32_t b = (e >= 0 && e < r.n_as) ? e : (int32_t)r.n_as;
        if (e >= r.n_as) *r.bad_id = 1;
        atomicAdd(&cnt[b], 1);
        scratch[p] = b;
    }
    __syncthreads();
    // exclusive scan of the experts' task counts: thread tid owns experts [tid per, tid per + per),
    // a wave scan by shuffles, then the 16 wave totals through LDS
    {
        const int64_t per = (nbk + kRouteThreads - 1) / kRouteThreads, e0 = tid * per;
        int32_t local = 0;
        for (int64_t k = 0; k < per; ++k)
            if (e0 + k < nbk) local += (cnt[e0 + k] + TC - 1) / TC;
        const int lane = tid & 63, wave = tid >> 6;
        int32_t x = local;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int32_t v = __shfl_up(x, d, 64);
            if (lane >= d) x += v;
        }
        if (lane == 63) s_wsum[wave] = x;
        __syncthreads();
        if (tid == 0) {
            int32_t acc = 0;
            for (int w = 0; w < kRouteThreads / 64; ++w) {
                const int32_t t = s_wsum[w];
                s_wsum[w] = acc;
                acc += t;
            }
            *ntasks = acc;
        }
        __syncthreads();
        int32_t excl = x - local + s_wsum[wave];
        for (int64_t k = 0; k < per; ++k)
            if (e0 + k < nbk) {
                tstart[e0 + k] = excl;
                excl += (cnt[e0 + k] + TC - 1) / TC;
            }
    }
    __syncthreads();
    // task headers (the invalid bucket's tasks: mat = -1, zero rows)
    for (int64_t e = tid; e < nbk; e += kRouteThreads) {
        const int32_t c = cnt[e];
        const int32_t nt = (c + TC - 1) / TC;
        for (int32_t k = 0; k < nt; ++k) {
            TaskOf<TC> & T = tasks[tstart[e] + k];
            T.mat = e < r.n_as ? (int32_t)(QMM_RED == 7 ? (e + 1) % r.n_as : e) : -1;   // (mutation 7: next expert)
            T.ncols = (c - k * TC) < TC ? (c - k * TC) : TC;
        }
    }
    __syncthreads();
    for (int64_t e = tid; e < nbk; e += kRouteThreads) cnt[e] = 0;
    __syncthreads();
    for (int64_t p = tid; p < npairs; p += kRouteThreads) {
        const int32_t b = scratch[p];
        const int64_t t = p / r.n_used, i = p % r.n_used;
        const int32_t slot = atomicAdd(&cnt[b], 1);
        TaskOf<TC> & T = tasks[tstart[b] + slot / TC];
        T.col[slot % TC] = b < r.n_as ? (int32_t)((i % r.ne11) + t * r.ne11) : 0;
        T.dst_off[slot % TC] = t * r.dst_nb2 + i * r.dst_nb1;
    }
}

template <int TC>
__global__ __launch_bounds__(kRouteThreads) void k_route(RouteArgs r, int32_t * __restrict__ scratch,
                                                         TaskOf<TC> * __restrict__ tasks, int32_t * __restrict__ ntasks) {
    extern __shared__ int32_t sm[];
    __shared__ int32_t s_wsum[kRouteThreads / 64];
    route_body<TC>(r, scratch, tasks, ntasks, sm, s_wsum);
}

// MUL_MAT_ID's two independent preparations in one launch: work-group 0 routes, the others
// quantize the activations (the q8_0 or q8_K pass of the quantization launch, no dst
// zeroing).  At decode both are a few microseconds of latency each; side by side the GEMV
// waits for the longer one instead of their sum.
template <int VDT, int TC>
__global__ __launch_bounds__(kRouteThreads) void k_quant_route(F32Cols src, int64_t K, int64_t ncols, ActBuf a,
                                                               RouteArgs r, int32_t * __restrict__ scratch,
                                                               TaskOf<TC> * __restrict__ tasks,
                                                               int32_t * __restrict__ ntasks) {
    extern __shared__ int32_t sm[];
    __shared__ int32_t s_wsum[kRouteThreads / 64];
    if (blockIdx.x == 0) {                                        // uniform
        route_body<TC>(r, scratch, tasks, ntasks, sm, s_wsum);
        return;
    }
    const int64_t t = (int64_t)(blockIdx.x - 1) * kRouteThreads + threadIdx.x;
    if (VDT == QMM_TYPE_Q8_0) quant_q8_0_at(src, K, ncols, a, t);
    else quant_q8_K_at(src, K, ncols, a, t);
}

// ---- the router: softmax -> top-k -> normalized weights ------------------------------------
// Role of the reference's fused router (kernel_topk_moe_softmax_norm, P09:899-1000), which
// replaces llama.cpp's gating chain SOFT_MAX, ARGSORT (desc), VIEW, GET_ROWS, SUM_ROWS, CLAMP,
// DIV (matched at P02:786-821); the selection here is a filter and a count, not repeated arg-max
// rounds.  One wave per token (a one-wave work-group); lane l holds the logits of the NPER
// consecutive experts [l NPER, (l + 1) NPER).  The order is the reference's: the float32 values
// e = exp(x - max) it ranks (P09:935-966), equal values to the lower expert, so two distinct
// logits whose float32 exp is equal tie (as ggml's SOFT_MAX -> ARGSORT ranks float32
// probabilities):
//  1. each e becomes a 32-bit key, its bits + 1 (e >= 0, so the bits are in e's order; an exp
//     that underflows to 0 still ranks above the padding); padding gets key 0;
//  2. the filter: tau0 = the k-th largest of the 64 lanes' largest keys, found most-significant
//     bit first (32 steps of one ballot).  The lanes holding the k largest maxima hold k keys
//     >= tau0, so every winner is >= tau0;
//  3. the candidates (keys >= tau0; usually a few more than k) go to LDS at the offsets of a
//     scan of the lanes' counts, in expert order;
//  4. each candidate counts the candidates ahead of it (larger key, or equal key and lower
//     expert): those with fewer than k ahead win, at that rank.
// Weights: exp(x - max) / sum over all experts (a wave sum), divided by the winners' sum, taken
// in rank order and clamped to [cmin, cmax].


// the sum over lanes 0 .. lane of v (inclusive), by shuffles
__device__ __forceinline__ int lane_scan(int v, int lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int u = __shfl_up(v, d, 64);
        if (lane >= d) v += u;
    }
    return v;
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d, 64);
    return v;
}

constexpr int kTopkMaxExperts = 1024;

template <int NPER>
__global__ __launch_bounds__(64) void k_topk(TopkArgs a) {
    __shared__ uint32_t cand_key[kTopkMaxExperts];
    __shared__ int cand_exp[kTopkMaxExperts];
    __shared__ float ranked_p[32];
    const int lane = threadIdx.x;
    const int64_t t = blockIdx.x;
    const float * x = reinterpret_cast<const float *>(a.logits + t * a.nbl1);
    const int e0 = lane * NPER, k = a.k;
    float v[NPER];
    uint32_t key[NPER];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
        v[j] = e0 + j < a.n_expert ? x[e0 + j] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    const float m = wave_max(mx);
    float part = 0.0f;
    uint32_t kmax = 0;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
        const bool live = e0 + j < a.n_expert;
        const float e = live ? expf(v[j] - m) : 0.0f;
        part += e;
        key[j] = live ? __builtin_bit_cast(uint32_t, e) + 1u : 0u;
        kmax = key[j] > kmax ? key[j] : kmax;
    }
    const float S = wave_sum_f(part);
    // 2. tau0: the largest value with at least k lane maxima at or above it
    uint32_t tau0 = 0;
    for (int b = 31; b >= 0; --b) {
        const uint32_t c = tau0 | (1u << b);
        if (__popcll(__ballot(kmax >= c)) >= k) tau0 = c;
    }
    // 3. the candidates into LDS, in expert order
    int nc = 0;
#pragma unroll
    for (int j = 0; j < NPER; ++j) nc += key[j] >= tau0;
    int slot = lane_scan(nc, lane) - nc;
    const int ncand = __shfl(slot + nc, 63, 64);
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
        if (key[j] >= tau0) {
            cand_key[slot] = key[j];
            cand_exp[slot] = e0 + j;
            ++slot;
        }
    }
    __syncthreads();
    // 4. each candidate's rank; the first k are the winners (their probabilities summed in
    // rank order below)
    int my_rank[kTopkMaxExperts / 64], my_exp[kTopkMaxExperts / 64];
    float my_p[kTopkMaxExperts / 64];
    int nmine = 0;
    for (int c = lane; c < ncand; c += 64) {
        const uint32_t ku = cand_key[c];
        const int ke = cand_exp[c];
        int r = 0;
        for (int i = 0; i < ncand && r < k; ++i) r += cand_key[i] > ku || (cand_key[i] == ku && cand_exp[i] < ke);
        if (r < k) {
            const float p = expf(x[ke] - m) / S;
            ranked_p[r] = p;
            my_rank[nmine] = r;
            my_exp[nmine] = ke;
            my_p[nmine] = p;
            ++nmine;
        }
    }
    __syncthreads();
    float wsum = 0.0f;
    for (int i = 0; i < k; ++i) wsum += ranked_p[i];               // uniform, in rank order
    const float cl = fminf(fmaxf(wsum, a.cmin), a.cmax);
    for (int q = 0; q < nmine; ++q) {
        reinterpret_cast<int32_t *>(a.ids + t * a.nbi1)[my_rank[q]] = my_exp[q];
        reinterpret_cast<float *>(a.w + t * a.nbw1)[my_rank[q]] = my_p[q] / cl;
    }
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
    if (a.shared) {
        const float g = *reinterpret_cast<const float *>(a.gate + t * a.gnb1);
        const float sg = 1.0f / (1.0f + expf(-g));
        y = y + *reinterpret_cast<const float *>(a.shared + t * a.snb1 + m * 4) * sg;
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
template <int TC>
hipError_t route_t(const RouteArgs & r, int32_t * scratch, TaskOf<TC> * tasks, int32_t * ntasks, hipStream_t s) {
    const size_t lds = (size_t)(r.n_as + 1) * 2 * sizeof(int32_t);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    k_route<TC><<<1, kRouteThreads, lds, s>>>(r, scratch, tasks, ntasks);
    return hipGetLastError();
}

template <int TC>
hipError_t quant_route_t(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, const RouteArgs & r,
                         int32_t * scratch, TaskOf<TC> * tasks, int32_t * ntasks, hipStream_t s) {
    const size_t lds = (size_t)(r.n_as + 1) * 2 * sizeof(int32_t);
    if (lds > 64 * 1024 || K <= 0 || ncols < 0 || a.ldk % 256 || a.ldk < K) return hipErrorInvalidValue;
    const int64_t nq = a.vdt == QMM_TYPE_Q8_0 ? ncols * (a.ldk / 4) : ncols * (a.ldk / 256) * 64;
    const int64_t grid = 1 + (nq + kRouteThreads - 1) / kRouteThreads;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    if (a.vdt == QMM_TYPE_Q8_0)
        k_quant_route<QMM_TYPE_Q8_0, TC><<<dim3((unsigned)grid), kRouteThreads, lds, s>>>(src, K, ncols, a, r, scratch,
                                                                                          tasks, ntasks);
    else
        k_quant_route<QMM_TYPE_Q8_K, TC><<<dim3((unsigned)grid), kRouteThreads, lds, s>>>(src, K, ncols, a, r, scratch,
                                                                                          tasks, ntasks);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_route(const RouteArgs & r, int32_t * scratch, GemvTask * tasks, int32_t * ntasks, hipStream_t s) {
    return route_t(r, scratch, tasks, ntasks, s);
}
hipError_t launch_route(const RouteArgs & r, int32_t * scratch, GemmUnit * units, int32_t * nunits, hipStream_t s) {
    return route_t(r, scratch, units, nunits, s);
}
hipError_t launch_quant_route(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, const RouteArgs & r,
                              int32_t * scratch, GemvTask * tasks, int32_t * ntasks, hipStream_t s) {
    return quant_route_t(src, K, ncols, a, r, scratch, tasks, ntasks, s);
}
hipError_t launch_quant_route(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, const RouteArgs & r,
                              int32_t * scratch, GemmUnit * units, int32_t * nunits, hipStream_t s) {
    return quant_route_t(src, K, ncols, a, r, scratch, units, nunits, s);
}

}  // namespace qmm
