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

namespace qmm {
namespace {

constexpr int kRouteThreads = 1024;

// one work-group of kRouteThreads; sm = [2 (n_as + 1)] ints of LDS, s_wsum = [kRouteThreads / 64]
__device__ __forceinline__ void route_body(const RouteArgs & r, int32_t * __restrict__ scratch,
                                           GemvTask * __restrict__ tasks, int32_t * __restrict__ ntasks,
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
            if (e0 + k < nbk) local += (cnt[e0 + k] + kMaxTaskCols - 1) / kMaxTaskCols;
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
                excl += (cnt[e0 + k] + kMaxTaskCols - 1) / kMaxTaskCols;
            }
    }
    __syncthreads();
    // task headers (the invalid bucket's tasks: mat = -1, zero rows)
    for (int64_t e = tid; e < nbk; e += kRouteThreads) {
        const int32_t c = cnt[e];
        const int32_t nt = (c + kMaxTaskCols - 1) / kMaxTaskCols;
        for (int32_t k = 0; k < nt; ++k) {
            GemvTask & T = tasks[tstart[e] + k];
            T.mat = e < r.n_as ? (int32_t)e : -1;
            T.ncols = (c - k * kMaxTaskCols) < kMaxTaskCols ? (c - k * kMaxTaskCols) : kMaxTaskCols;
        }
    }
    __syncthreads();
    for (int64_t e = tid; e < nbk; e += kRouteThreads) cnt[e] = 0;
    __syncthreads();
    for (int64_t p = tid; p < npairs; p += kRouteThreads) {
        const int32_t b = scratch[p];
        const int64_t t = p / r.n_used, i = p % r.n_used;
        const int32_t slot = atomicAdd(&cnt[b], 1);
        GemvTask & T = tasks[tstart[b] + slot / kMaxTaskCols];
        T.col[slot % kMaxTaskCols] = b < r.n_as ? (int32_t)((i % r.ne11) + t * r.ne11) : 0;
        T.dst_off[slot % kMaxTaskCols] = t * r.dst_nb2 + i * r.dst_nb1;
    }
}

__global__ __launch_bounds__(kRouteThreads) void k_route(RouteArgs r, int32_t * __restrict__ scratch,
                                                         GemvTask * __restrict__ tasks, int32_t * __restrict__ ntasks) {
    extern __shared__ int32_t sm[];
    __shared__ int32_t s_wsum[kRouteThreads / 64];
    route_body(r, scratch, tasks, ntasks, sm, s_wsum);
}

// MUL_MAT_ID's two independent preparations in one launch: work-group 0 routes, the others
// quantize the activations (the q8_0 or q8_K pass of the quantization launch, no dst
// zeroing).  At decode both are a few microseconds of latency each; side by side the GEMV
// waits for the longer one instead of their sum.
template <int VDT>
__global__ __launch_bounds__(kRouteThreads) void k_quant_route(F32Cols src, int64_t K, int64_t ncols, ActBuf a,
                                                               RouteArgs r, int32_t * __restrict__ scratch,
                                                               GemvTask * __restrict__ tasks,
                                                               int32_t * __restrict__ ntasks) {
    extern __shared__ int32_t sm[];
    __shared__ int32_t s_wsum[kRouteThreads / 64];
    if (blockIdx.x == 0) {                                        // uniform
        route_body(r, scratch, tasks, ntasks, sm, s_wsum);
        return;
    }
    const int64_t t = (int64_t)(blockIdx.x - 1) * kRouteThreads + threadIdx.x;
    if (VDT == QMM_TYPE_Q8_0) quant_q8_0_at(src, K, ncols, a, t);
    else quant_q8_K_at(src, K, ncols, a, t);
}

// ---- the router: softmax -> top-k -> normalized weights ------------------------------------
// Role of the reference's fused router (kernel_topk_moe_softmax_norm, P09:899-1000), which
// replaces llama.cpp's gating chain SOFT_MAX, ARGSORT (desc), VIEW, GET_ROWS, SUM_ROWS, CLAMP,
// DIV (matched at P02:786-821); the selection here is a threshold search, not repeated arg-max
// rounds.  One wave per token (a one-wave work-group); lane l holds the logits of the NPER
// consecutive experts [l NPER, (l + 1) NPER).  Softmax is monotone, so the winners are the k
// largest logits, equal logits ordered by expert (the order of the probabilities, which the
// float32 exp could otherwise merge into ties):
//  1. each logit becomes an order-preserving 32-bit key; padding lanes get key 0, below every
//     real key;
//  2. the k-th largest key tau is found most-significant bit first: 32 steps, each counting the
//     keys at or above a candidate with one ballot per register (the count is uniform);
//  3. every key above tau wins, and of the keys equal to tau the lowest experts, counted in
//     expert order by an exclusive scan of the lanes' tie counts, until there are k;
//  4. the k winners go to LDS at the offsets of a scan of the lanes' win counts, and each of
//     the first k lanes counts the winners ahead of its own (larger key, or equal key and lower
//     expert): its rank in the output.
// Weights: exp(x - max) / sum over all experts (a wave sum), divided by the winners' sum, taken
// in rank order and clamped to [cmin, cmax].

// a float's bits as an unsigned key with the float's order (-0 as +0: equal floats, equal keys)
__device__ __forceinline__ uint32_t order_key(float x) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x == 0.0f ? 0.0f : x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

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

// number of register values of the wave with pred true (uniform)
template <int NPER, typename F>
__device__ __forceinline__ int wave_count(F pred) {
    int c = 0;
#pragma unroll
    for (int j = 0; j < NPER; ++j) c += __popcll(__ballot(pred(j)));
    return c;
}

template <int NPER>
__global__ __launch_bounds__(64) void k_topk(TopkArgs a) {
    __shared__ uint32_t win_key[32];
    __shared__ int win_exp[32];
    __shared__ float win_p[32], ranked_p[32];
    const int lane = threadIdx.x;
    const int64_t t = blockIdx.x;
    const float * x = reinterpret_cast<const float *>(a.logits + t * a.nbl1);
    const int e0 = lane * NPER, k = a.k;
    float v[NPER];
    uint32_t key[NPER];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
        const bool live = e0 + j < a.n_expert;
        v[j] = live ? x[e0 + j] : -INFINITY;
        key[j] = live ? order_key(v[j]) : 0u;
        mx = fmaxf(mx, v[j]);
    }
    const float m = wave_max(mx);
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < NPER; ++j)
        if (e0 + j < a.n_expert) part += expf(v[j] - m);
    const float S = wave_sum_f(part);
    // 2. tau: the largest key with at least k keys at or above it
    uint32_t tau = 0;
    for (int b = 31; b >= 0; --b) {
        const uint32_t cand = tau | (1u << b);
        if (wave_count<NPER>([&](int j) { return key[j] >= cand; }) >= k) tau = cand;
    }
    // 3. winners: keys above tau, then ties at tau in expert order
    const int need = k - wave_count<NPER>([&](int j) { return key[j] > tau; });   // >= 1
    int ties = 0;
#pragma unroll
    for (int j = 0; j < NPER; ++j) ties += key[j] == tau;
    int tie_rank = lane_scan(ties, lane) - ties;                  // ties at lower experts
    bool win[NPER];
    int nwin = 0;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
        win[j] = key[j] > tau;
        if (key[j] == tau) win[j] = tie_rank++ < need;
        nwin += win[j];
    }
    // 4. compaction into LDS, then each winner's rank
    int slot = lane_scan(nwin, lane) - nwin;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
        if (win[j]) {
            win_key[slot] = key[j];
            win_exp[slot] = e0 + j;
            win_p[slot] = expf(v[j] - m) / S;
            ++slot;
        }
    }
    __syncthreads();
    int rank = 0, my_exp = 0;
    float my_p = 0.0f;
    if (lane < k) {
        const uint32_t ku = win_key[lane];
        my_exp = win_exp[lane];
        my_p = win_p[lane];
        for (int i = 0; i < k; ++i) rank += win_key[i] > ku || (win_key[i] == ku && win_exp[i] < my_exp);
        ranked_p[rank] = my_p;
    }
    __syncthreads();
    float wsum = 0.0f;
    for (int i = 0; i < k; ++i) wsum += ranked_p[i];              // uniform, in rank order
    if (lane < k) {
        const float c = fminf(fmaxf(wsum, a.cmin), a.cmax);
        reinterpret_cast<int32_t *>(a.ids + t * a.nbi1)[rank] = my_exp;
        reinterpret_cast<float *>(a.w + t * a.nbw1)[rank] = my_p / c;
    }
}

// ---- the combine: dst[:, t] = sum_j w[j, t] experts[:, j, t] (+ shared[:, t] sigmoid(g[t]))
// in llama.cpp's order: the products rounded, added slot by slot, then the gated shared
// expert added (contraction off: ggml-cpu's MUL then ADDs round every product).
__global__ __launch_bounds__(256) void k_combine(CombineArgs a) {
#pragma clang fp contract(off)
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.M * a.T) return;
    const int64_t t = idx / a.M, m = idx - t * a.M;
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
    if (a.M < 1 || a.T < 1 || a.k < 1 || a.M * a.T >= ((int64_t)1 << 40)) return hipErrorInvalidValue;
    k_combine<<<dim3((unsigned)((a.M * a.T + 255) / 256)), 256, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_route(const RouteArgs & r, int32_t * scratch, GemvTask * tasks, int32_t * ntasks, hipStream_t s) {
    const size_t lds = (size_t)(r.n_as + 1) * 2 * sizeof(int32_t);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    k_route<<<1, kRouteThreads, lds, s>>>(r, scratch, tasks, ntasks);
    return hipGetLastError();
}

hipError_t launch_quant_route(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, const RouteArgs & r,
                              int32_t * scratch, GemvTask * tasks, int32_t * ntasks, hipStream_t s) {
    const size_t lds = (size_t)(r.n_as + 1) * 2 * sizeof(int32_t);
    if (lds > 64 * 1024 || K <= 0 || ncols < 0 || a.ldk % 256 || a.ldk < K) return hipErrorInvalidValue;
    const int64_t nq = a.vdt == QMM_TYPE_Q8_0 ? ncols * (a.ldk / 4) : ncols * (a.ldk / 256) * 64;
    const int64_t grid = 1 + (nq + kRouteThreads - 1) / kRouteThreads;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    if (a.vdt == QMM_TYPE_Q8_0)
        k_quant_route<QMM_TYPE_Q8_0><<<dim3((unsigned)grid), kRouteThreads, lds, s>>>(src, K, ncols, a, r, scratch, tasks, ntasks);
    else
        k_quant_route<QMM_TYPE_Q8_K><<<dim3((unsigned)grid), kRouteThreads, lds, s>>>(src, K, ncols, a, r, scratch, tasks, ntasks);
    return hipGetLastError();
}

}  // namespace qmm
