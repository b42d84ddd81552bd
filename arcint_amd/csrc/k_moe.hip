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
// writes dst + t * nb2 + i * nb1 (P01:3916-3922); a negative or out-of-range
// id writes a zero row (P02:98-103): such pairs go to one more bucket whose
// tasks (mat = -1) the GEMV turns into zero rows, so the route writes no dst
// and one route serves every product that shares the ids.
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

// ---- the router: softmax -> top-k -> normalized weights, one wave per token ----------
// Role of the reference's kernel_topk_moe_softmax_norm (P09:899-1000), which replaces
// llama.cpp's gating chain SOFT_MAX, ARGSORT (desc), VIEW, GET_ROWS, SUM_ROWS, CLAMP, DIV
// (matched at P02:786-821).  Lane l holds the logits of experts l + 64 j, j < NPER.  The max
// and the sum of exp(x - max) are wave reductions; each of the k rounds picks the largest
// unselected exp(x - max) over the wave (ties: the lower expert) by DPP reductions.  The
// weights are the picked exp(x - max) / sum, divided by their own sum clamped to [cmin, cmax].
constexpr int kTopkWaves = 4;                   // tokens per work-group

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d, 64);
    return v;
}

template <int NPER>
__global__ __launch_bounds__(64 * kTopkWaves) void k_topk(TopkArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t t = (int64_t)blockIdx.x * kTopkWaves + wave;
    if (t >= a.n_tok) return;                                     // whole waves
    const float * x = reinterpret_cast<const float *>(a.logits + t * a.nbl1);
    float p[NPER];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
        const int i = lane + 64 * j;
        p[j] = i < a.n_expert ? x[i] : -INFINITY;
        m = fmaxf(m, p[j]);
    }
    m = wave_max(m);
    float sl = 0.0f;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
        const int i = lane + 64 * j;
        p[j] = i < a.n_expert ? expf(p[j] - m) : -1.0f;          // -1: no expert (never picked)
        if (i < a.n_expert) sl += p[j];
    }
    const float s = wave_sum_f(sl);
    uint32_t sel = 0;                                             // bit j: p[j] picked
    float wsum = 0.0f, my_w = 0.0f;
    int my_id = 0;
    for (int r = 0; r < a.k; ++r) {                               // uniform
        float bv = -1.0f;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < NPER; ++j) {
            if (!(sel >> j & 1u) && p[j] > bv) {                  // j ascending: ties keep the lower expert
                bv = p[j];
                bi = lane + 64 * j;
            }
        }
        // the wave's largest value (DPP row reductions, four readlanes), then the lowest expert
        // among the lanes holding it
        const float gv = wave_max(bv);
        bi = wave_min_i(bv == gv ? bi : 0x7fffffff);
        bv = gv;
        const float wr = bv / s;
        wsum += wr;
        if (lane == r) {
            my_w = wr;
            my_id = bi;
        }
        if ((bi & 63) == lane && bi < a.n_expert) sel |= 1u << (bi >> 6);
    }
    if (lane < a.k) {
        const float c = fminf(fmaxf(wsum, a.cmin), a.cmax);
        reinterpret_cast<int32_t *>(a.ids + t * a.nbi1)[lane] = my_id;
        reinterpret_cast<float *>(a.w + t * a.nbw1)[lane] = my_w / c;
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
    const dim3 g((unsigned)((a.n_tok + kTopkWaves - 1) / kTopkWaves)), b(64 * kTopkWaves);
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
