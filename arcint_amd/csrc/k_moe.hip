// k_moe.hip - MUL_MAT_ID routing on gfx950.
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
// id writes a zero row (P02:98-103).
#include "qmm_device.h"

namespace qmm {
namespace {

constexpr int kRouteThreads = 1024;

__global__ __launch_bounds__(kRouteThreads) void k_route(RouteArgs r, int32_t * __restrict__ scratch,
                                                         GemvTask * __restrict__ tasks, int32_t * __restrict__ ntasks,
                                                         float * __restrict__ dst, int64_t M) {
    extern __shared__ int32_t sm[];
    int32_t * cnt = sm;                 // [n_as] pair count, later the fill cursor
    int32_t * tstart = sm + r.n_as;     // [n_as] first task of each expert
    __shared__ int32_t s_wsum[kRouteThreads / 64];
    const int tid = threadIdx.x;
    const int64_t npairs = r.n_used * r.T;
    for (int64_t e = tid; e < r.n_as; e += kRouteThreads) cnt[e] = 0;
    __syncthreads();
    for (int64_t p = tid; p < npairs; p += kRouteThreads) {
        const int64_t t = p / r.n_used, i = p % r.n_used;
        const int32_t e = *reinterpret_cast<const int32_t *>(reinterpret_cast<const char *>(r.ids) + t * r.ids_nb1 + i * r.ids_nb0);
        if (e >= 0 && e < r.n_as) atomicAdd(&cnt[e], 1);
        scratch[p] = e;
    }
    __syncthreads();
    // exclusive scan of the experts' task counts: thread tid owns experts [tid per, tid per + per),
    // a wave scan by shuffles, then the 16 wave totals through LDS
    {
        const int64_t per = (r.n_as + kRouteThreads - 1) / kRouteThreads, e0 = tid * per;
        int32_t local = 0;
        for (int64_t k = 0; k < per; ++k)
            if (e0 + k < r.n_as) local += (cnt[e0 + k] + kMaxTaskCols - 1) / kMaxTaskCols;
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
            if (e0 + k < r.n_as) {
                tstart[e0 + k] = excl;
                excl += (cnt[e0 + k] + kMaxTaskCols - 1) / kMaxTaskCols;
            }
    }
    __syncthreads();
    // task headers
    for (int64_t e = tid; e < r.n_as; e += kRouteThreads) {
        const int32_t c = cnt[e];
        const int32_t nt = (c + kMaxTaskCols - 1) / kMaxTaskCols;
        for (int32_t k = 0; k < nt; ++k) {
            GemvTask & T = tasks[tstart[e] + k];
            T.mat = (int32_t)e;
            T.ncols = (c - k * kMaxTaskCols) < kMaxTaskCols ? (c - k * kMaxTaskCols) : kMaxTaskCols;
        }
    }
    __syncthreads();
    for (int64_t e = tid; e < r.n_as; e += kRouteThreads) cnt[e] = 0;
    __syncthreads();
    for (int64_t p = tid; p < npairs; p += kRouteThreads) {
        const int32_t e = scratch[p];
        const int64_t t = p / r.n_used, i = p % r.n_used;
        const int64_t doff = t * r.dst_nb2 + i * r.dst_nb1;
        if (e >= 0 && e < r.n_as) {
            const int32_t slot = atomicAdd(&cnt[e], 1);
            GemvTask & T = tasks[tstart[e] + slot / kMaxTaskCols];
            T.col[slot % kMaxTaskCols] = (int32_t)((i % r.ne11) + t * r.ne11);
            T.dst_off[slot % kMaxTaskCols] = doff;
        } else {
            for (int64_t m = 0; m < M; ++m) dst[doff + m] = 0.0f;
        }
    }
}

}  // namespace

hipError_t launch_route(const RouteArgs & r, int32_t * scratch, GemvTask * tasks, int32_t * ntasks,
                        float * dst, int64_t M, hipStream_t s) {
    const size_t lds = (size_t)r.n_as * 2 * sizeof(int32_t);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    k_route<<<1, kRouteThreads, lds, s>>>(r, scratch, tasks, ntasks, dst, M);
    return hipGetLastError();
}

}  // namespace qmm
