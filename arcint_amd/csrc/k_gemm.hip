// k_gemm.hip - prefill GEMM (N >= 16 columns) on gfx950 int8 MFMA.
//
// Role of the reference's int8 prefill GEMMs (kernel_mul_mm_kq2d_q4_0_i8 and
// kernel_mul_mm_kq2d_q4_K_i8, P0099:362-455 and P01:1862-2024; the SG8 forms
// P0099:456-631, P0102:151-283), redesigned for CDNA4 and for ggml-cpu's
// numerics:
//  * the activations are the pre-pass's q8_0 / q8_K codes (bit-exact with
//    ggml-cpu's from_float) and serve as the MFMA A operand straight from
//    global memory: tokens are the 16 rows of a v_mfma_i32_16x16x32_i8 tile,
//    one 8-byte load per lane per 32-element K granule;
//  * the weights are the B operand: every lane turns 8 bytes of a weight
//    plane into 8 signed int8 codes in registers (nibble split, Q4_0's -8,
//    Q6_K's 6-bit assembly and -32, the IQ4 codebook by byte permutes), so
//    the int32 result of each MFMA is the exact integer dot of one
//    (sub-)block, as in ggml_vec_dot_*;
//  * per-block scaling stays on the VALU in the lane that holds the MFMA
//    result: Q4_0 / Q8_0 add int * (d_w * d_x) per 32-block; Q4_K / IQ4_XS /
//    Q6_K multiply by the integer sub-block scale into an int32 super-block
//    sum (the Q4_K min term is a second MFMA against the replicated 6-bit
//    mins, accumulated over the super-block) and add one float term per
//    256 weights;
//  * each wave owns 16*GT tokens x 16*GR weight rows, a work-group 2 x 2
//    waves; loads for granule k+1 are issued before granule k is used, and
//    every load is unconditional (clamped addresses) so the waits are exact;
//  * tiles are numbered so that the work-groups sharing one weight-row tile
//    land on the same XCD (its L2 serves the repeats).
// MFMA output layout (verified on the device): lane l holds rows 4*(l/16)+r,
// r < 4, of column l % 16.
#include "qmm_device.h"

#include <hip/hip_ext.h>

#include <algorithm>
#include <cstdlib>

namespace qmm {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

struct GemmParams {
    WView w;
    int64_t M, K, N;    // M, K repeat w.M, w.K
    const int8_t * codes;   // activation codes [ncols][ldk]
    int64_t ldk;
    const float * dT;       // activation scales [K / BS][ldT]
    int64_t ldT;
    int64_t ntiles, tiles_n, chunk;
    GemmBatch bt;
    float * dst;
};

__device__ __forceinline__ uint32_t sub8(uint32_t v, uint32_t k) {   // bytewise v - k, v in [0, 128), k < 128
    return ((v | 0x80808080u) - k) ^ 0x80808080u;
}

template <int TYPE> struct GW;

// Q4_0: granule = block kg; lane group g takes qs bytes 8(g&1)..+8, nibble g>>1
template <> struct GW<QMM_TYPE_Q4_0> {
    static constexpr int BS = 32;
    struct R { uint2 q; uint32_t d; };
    __device__ static void load(R & r, const uint8_t * tb, int rr, size_t tgs, int kg, int g) {
        const uint8_t * t = tb + (size_t)(kg >> 3) * tgs + rr * 16;
        const int p = kg & 7;
        r.q = *reinterpret_cast<const uint2 *>(t + p * kChunk + 8 * (g & 1));
        r.d = *reinterpret_cast<const uint16_t *>(t + 8 * kChunk + 2 * p);
    }
    __device__ static long bop(const R & r, int g) {
        const int sh = 4 * (g >> 1);
        const uint32_t lo = sub8((r.q.x >> sh) & 0x0F0F0F0Fu, 0x08080808u);
        const uint32_t hi = sub8((r.q.y >> sh) & 0x0F0F0F0Fu, 0x08080808u);
        return (long)(((uint64_t)hi << 32) | lo);
    }
};

// Q8_0: granule = block kg; lane group g takes qs bytes 8g..8g+7
template <> struct GW<QMM_TYPE_Q8_0> {
    static constexpr int BS = 32;
    struct R { uint2 q; uint32_t d; };
    __device__ static void load(R & r, const uint8_t * tb, int rr, size_t tgs, int kg, int g) {
        const uint8_t * t = tb + (size_t)(kg >> 3) * tgs + rr * 16;
        const int p = kg & 7;
        r.q = *reinterpret_cast<const uint2 *>(t + (2 * p + (g >> 1)) * kChunk + 8 * (g & 1));
        r.d = *reinterpret_cast<const uint16_t *>(t + 16 * kChunk + 2 * p);
    }
    __device__ static long bop(const R & r, int) { return (long)(((uint64_t)r.q.y << 32) | r.q.x); }
};

// Q4_K: granule = sub-block j = kg % 8 of super-block kg / 8 (chunk c = j/2,
// nibble j%2); lane group g takes qs bytes 32c+8g..+8; header per super-block
template <> struct GW<QMM_TYPE_Q4_K> {
    static constexpr int BS = 256;
    struct R { uint2 q; uint4 h; };
    __device__ static void load(R & r, const uint8_t * tb, int rr, size_t tgs, int kg, int g) {
        const uint8_t * t = tb + (size_t)(kg >> 3) * tgs + rr * 16;
        const int j = kg & 7;
        r.q = *reinterpret_cast<const uint2 *>(t + (2 * (j >> 1) + (g >> 1)) * kChunk + 8 * (g & 1));
        r.h = *reinterpret_cast<const uint4 *>(t + 8 * kChunk);
    }
    __device__ static long bop(const R & r, int kg) {
        const int sh = 4 * (kg & 1);
        const uint32_t lo = (r.q.x >> sh) & 0x0F0F0F0Fu, hi = (r.q.y >> sh) & 0x0F0F0F0Fu;
        return (long)(((uint64_t)hi << 32) | lo);
    }
    // 6-bit scale and min of sub-block j (get_scale_min_k4, P01:2164-2176)
    __device__ static void scale_min(const R & r, int j, int & sc, int & m) {
        const int b = 8 * (j & 3);
        if (j < 4) {
            sc = (r.h.y >> b) & 63;
            m = (r.h.z >> b) & 63;
        } else {
            sc = ((r.h.w >> b) & 0xF) | (((r.h.y >> b) >> 6 & 3) << 4);
            m = ((r.h.w >> b) >> 4 & 0xF) | (((r.h.z >> b) >> 6 & 3) << 4);
        }
    }
};

// IQ4_XS: granule = sub-block ib = kg % 8; lane group g takes qs bytes
// 16ib+8(g&1)..+8, nibble g>>1, through the codebook
template <> struct GW<QMM_TYPE_IQ4_XS> {
    static constexpr int BS = 256;
    struct R { uint2 q; uint2 h; };
    __device__ static void load(R & r, const uint8_t * tb, int rr, size_t tgs, int kg, int g) {
        const uint8_t * t = tb + (size_t)(kg >> 3) * tgs;
        const int ib = kg & 7;
        r.q = *reinterpret_cast<const uint2 *>(t + ib * kChunk + rr * 16 + 8 * (g & 1));
        r.h = *reinterpret_cast<const uint2 *>(t + 8 * kChunk + rr * 8);
    }
    __device__ static long bop(const R & r, int g) {
        const int sh = 4 * (g >> 1);
        const uint32_t lo = iq4_lookup((r.q.x >> sh) & 0x0F0F0F0Fu), hi = iq4_lookup((r.q.y >> sh) & 0x0F0F0F0Fu);
        return (long)(((uint64_t)hi << 32) | lo);
    }
    __device__ static int ls(const R & r, int ib) {
        return (int)(((r.h.y >> (4 * ib)) & 0xF) | (((r.h.x >> (16 + 2 * ib)) & 3) << 4)) - 32;
    }
};

// Q6_K: granule = quarter gq of half n of super-block kg / 8 (qi = kg % 8 =
// 4n + gq): weights 128n + 32gq + l, l = 8g..8g+7 for lane group g, so lane
// groups 0-1 hold scale group 8n+2gq and 2-3 hold 8n+2gq+1
template <> struct GW<QMM_TYPE_Q6_K> {
    static constexpr int BS = 256;
    struct R { uint2 ql, qh; uint4 sc; uint32_t d; };
    __device__ static void load(R & r, const uint8_t * tb, int rr, size_t tgs, int kg, int g) {
        const uint8_t * t = tb + (size_t)(kg >> 3) * tgs;
        const int qi = kg & 7, n = qi >> 2, gq = qi & 3;
        const uint8_t * tr = t + rr * 16;
        r.ql = *reinterpret_cast<const uint2 *>(tr + (4 * n + 2 * (gq & 1) + (g >> 1)) * kChunk + 8 * (g & 1));
        r.qh = *reinterpret_cast<const uint2 *>(tr + (8 + 2 * n + (g >> 1)) * kChunk + 8 * (g & 1));
        r.sc = *reinterpret_cast<const uint4 *>(tr + 12 * kChunk);
        r.d = *reinterpret_cast<const uint16_t *>(t + 13 * kChunk + rr * 2);
    }
    __device__ static long bop(const R & r, int kg) {
        const int gq = kg & 3, shl = 4 * (gq >> 1), shh = 2 * gq;
        const uint32_t lo = ((r.ql.x >> shl) & 0x0F0F0F0Fu) | (((r.qh.x >> shh) & 0x03030303u) << 4);
        const uint32_t hi = ((r.ql.y >> shl) & 0x0F0F0F0Fu) | (((r.qh.y >> shh) & 0x03030303u) << 4);
        return (long)(((uint64_t)sub8(hi, 0x20202020u) << 32) | sub8(lo, 0x20202020u));
    }
    __device__ static int scale(const R & r, int idx) {   // int8 scales[idx]
        const uint32_t wd = idx < 4 ? r.sc.x : idx < 8 ? r.sc.y : idx < 12 ? r.sc.z : r.sc.w;
        return (int)(int8_t)((wd >> (8 * (idx & 3))) & 0xff);
    }
};

template <int TYPE, int GT, int GR>
__global__ __launch_bounds__(kThreads) void k_gemm(GemmParams p) {
    using T = GW<TYPE>;
    using R = typename T::R;
    constexpr bool KQ = TYPE == QMM_TYPE_Q4_K || TYPE == QMM_TYPE_Q6_K || TYPE == QMM_TYPE_IQ4_XS;
    const int bid = blockIdx.x;
    const int64_t logical = (int64_t)(bid & 7) * p.chunk + (bid >> 3);
    if (logical >= p.ntiles) return;                       // uniform
    const int64_t n_tile = logical % p.tiles_n, m_tile = logical / p.tiles_n;
    const int64_t bz = blockIdx.y;
    const int64_t i2 = bz % p.bt.ne12, i3 = bz / p.bt.ne12;
    const int64_t mat = i2 / p.bt.r2 + (i3 / p.bt.r3) * p.bt.ne02;
    const int64_t col0 = bz * p.N;
    float * dst = p.dst + i2 * p.bt.d_nb2 + i3 * p.bt.d_nb3;

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g = lane >> 4, c16 = lane & 15;
    const int64_t n0 = n_tile * (32 * GT) + (wave & 1) * (16 * GT);
    const int64_t m0 = m_tile * (32 * GR) + (wave >> 1) * (16 * GR);
    const int64_t N = p.N, M = p.M, K = p.K;

    const int8_t * arow[GT];                               // A operand: token rows
    int64_t dq[GT];                                        // column of the lane's first of 4 tokens in dT
#pragma unroll
    for (int t = 0; t < GT; ++t) {
        const int64_t n = n0 + 16 * t + c16;
        arow[t] = p.codes + (col0 + (n < N ? n : N - 1)) * p.ldk + 8 * g;
        dq[t] = col0 + n0 + 16 * t + 4 * g;               // < ncols + 61 <= ldT - 3 (64 columns of padding)
    }
    const uint8_t * wtb[GR];                               // B operand: weight rows (tile base, row in tile)
    int wrr[GR];
#pragma unroll
    for (int s = 0; s < GR; ++s) {
        const int64_t m0c = m0 + 16 * s + c16, m = m0c < M ? m0c : M - 1;
        wtb[s] = tile_group(p.w, mat, m / kTileRows, 0);
        wrr[s] = (int)(m % kTileRows);
    }
    const size_t tgs = (size_t)p.w.tg;

    const int nk = (int)(K / 32);
    float out[GT][GR][4];
    int acc[GT][GR][4];
    v4i accm[GT][GR];
    const v4i zero = { 0, 0, 0, 0 };
#pragma unroll
    for (int t = 0; t < GT; ++t)
#pragma unroll
        for (int s = 0; s < GR; ++s) {
            accm[t][s] = zero;
#pragma unroll
            for (int r = 0; r < 4; ++r) { out[t][s][r] = 0.0f; acc[t][s][r] = 0; }
        }

    long A0[GT], A1[GT];
    R W0[GR], W1[GR];
    float4 X0[GT], X1[GT];
    auto load = [&](int kg, long * A, R * W, float4 * X) {
#pragma unroll
        for (int t = 0; t < GT; ++t) A[t] = *reinterpret_cast<const long *>(arow[t] + (int64_t)kg * 32);
#pragma unroll
        for (int s = 0; s < GR; ++s) T::load(W[s], wtb[s], wrr[s], tgs, kg, g);
        const int64_t kb = (int64_t)kg * 32 / T::BS;
#pragma unroll
        for (int t = 0; t < GT; ++t) {                     // 4 dwords: col0 need not be a multiple of 4
            const float * xp = p.dT + kb * p.ldT + dq[t];
            X[t] = make_float4(xp[0], xp[1], xp[2], xp[3]);
        }
    };
    auto compute = [&](int kg, const long * A, const R * W, const float4 * X) {
        if constexpr (TYPE == QMM_TYPE_Q4_0 || TYPE == QMM_TYPE_Q8_0) {
#pragma unroll
            for (int s = 0; s < GR; ++s) {
                const long B = T::bop(W[s], g);
                const float dw = h2f(W[s].d);
#pragma unroll
                for (int t = 0; t < GT; ++t) {
                    const v4i D = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[t], B, zero, 0, 0, 0);
                    const float xs[4] = { X[t].x, X[t].y, X[t].z, X[t].w };
#pragma unroll
                    for (int r = 0; r < 4; ++r) out[t][s][r] += (float)D[r] * (dw * xs[r]);
                }
            }
        } else if constexpr (TYPE == QMM_TYPE_Q4_K) {
            const int j = kg & 7;
#pragma unroll
            for (int s = 0; s < GR; ++s) {
                const long B = T::bop(W[s], j);
                int sc, mn;
                T::scale_min(W[s], j, sc, mn);
                const long Bm = (long)((uint64_t)(uint32_t)mn * 0x0101010101010101ull);
#pragma unroll
                for (int t = 0; t < GT; ++t) {
                    const v4i D = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[t], B, zero, 0, 0, 0);
                    accm[t][s] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[t], Bm, accm[t][s], 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[t][s][r] += sc * D[r];
                }
            }
            if (j == 7) {                                  // end of the super-block (uniform)
#pragma unroll
                for (int s = 0; s < GR; ++s) {
                    const float d = h2f(W[s].h.x), dmin = h2f(W[s].h.x >> 16);
#pragma unroll
                    for (int t = 0; t < GT; ++t) {
                        const float xs[4] = { X[t].x, X[t].y, X[t].z, X[t].w };
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            out[t][s][r] += xs[r] * (d * (float)acc[t][s][r] - dmin * (float)accm[t][s][r]);
                            acc[t][s][r] = 0;
                        }
                        accm[t][s] = zero;
                    }
                }
            }
        } else if constexpr (TYPE == QMM_TYPE_IQ4_XS) {
            const int ib = kg & 7;
#pragma unroll
            for (int s = 0; s < GR; ++s) {
                const long B = T::bop(W[s], g);
                const int ls = T::ls(W[s], ib);
#pragma unroll
                for (int t = 0; t < GT; ++t) {
                    const v4i D = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[t], B, zero, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[t][s][r] += ls * D[r];
                }
            }
            if (ib == 7) {
#pragma unroll
                for (int s = 0; s < GR; ++s) {
                    const float d = h2f(W[s].h.x);
#pragma unroll
                    for (int t = 0; t < GT; ++t) {
                        const float xs[4] = { X[t].x, X[t].y, X[t].z, X[t].w };
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            out[t][s][r] += (d * xs[r]) * (float)acc[t][s][r];
                            acc[t][s][r] = 0;
                        }
                    }
                }
            }
        } else {                                           // Q6_K
            const int qi = kg & 7, n = qi >> 2, gq = qi & 3;
#pragma unroll
            for (int s = 0; s < GR; ++s) {
                const long B = T::bop(W[s], gq);
                const long B0 = g < 2 ? B : 0, B1 = g < 2 ? 0 : B;
                const int sc0 = T::scale(W[s], 8 * n + 2 * gq), sc1 = T::scale(W[s], 8 * n + 2 * gq + 1);
#pragma unroll
                for (int t = 0; t < GT; ++t) {
                    const v4i D0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[t], B0, zero, 0, 0, 0);
                    const v4i D1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[t], B1, zero, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[t][s][r] += sc0 * D0[r] + sc1 * D1[r];
                }
            }
            if (qi == 7) {
#pragma unroll
                for (int s = 0; s < GR; ++s) {
                    const float d = h2f(W[s].d);
#pragma unroll
                    for (int t = 0; t < GT; ++t) {
                        const float xs[4] = { X[t].x, X[t].y, X[t].z, X[t].w };
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            out[t][s][r] += (d * xs[r]) * (float)acc[t][s][r];
                            acc[t][s][r] = 0;
                        }
                    }
                }
            }
        }
        (void)KQ;
    };

    load(0, A0, W0, X0);
    for (int kg = 0; kg < nk; kg += 2) {
        load(kg + 1 < nk ? kg + 1 : nk - 1, A1, W1, X1);
        compute(kg, A0, W0, X0);
        load(kg + 2 < nk ? kg + 2 : nk - 1, A0, W0, X0);
        if (kg + 1 < nk) compute(kg + 1, A1, W1, X1);      // uniform
    }

#pragma unroll
    for (int t = 0; t < GT; ++t)
#pragma unroll
        for (int s = 0; s < GR; ++s) {
            const int64_t m = m0 + 16 * s + c16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t n = n0 + 16 * t + 4 * g + r;
                if (n < N && m < M) dst[n * p.bt.d_nb1 + m] = out[t][s][r];
            }
        }
}

template <int TYPE, int GT, int GR>
hipError_t launch_t(GemmParams p, int64_t nbatch, hipStream_t s, const KTime * kt) {
    const int64_t tiles_m = (p.M + 32 * GR - 1) / (32 * GR);
    p.tiles_n = (p.N + 32 * GT - 1) / (32 * GT);
    p.ntiles = tiles_m * p.tiles_n;
    p.chunk = (p.ntiles + 7) / 8;
    const int64_t grid = p.chunk * 8;
    if (grid > 0x7fffffff || nbatch > 65535) return hipErrorInvalidValue;
    const dim3 g((unsigned)grid, (unsigned)nbatch);
    if (kt) hipExtLaunchKernelGGL(k_gemm<TYPE, GT, GR>, g, dim3(kThreads), 0u, s, kt->start, kt->stop, 0, p);
    else k_gemm<TYPE, GT, GR><<<g, kThreads, 0, s>>>(p);
    return hipGetLastError();
}

}  // namespace

// QMM_GEMM_V1=1 keeps every type on the 16x16x32 kernel below
bool gemm_uses_v2(int type) {
    static const bool v1 = [] {
        const char * e = getenv("QMM_GEMM_V1");
        return e && atoi(e) != 0;
    }();
    return !v1 && gemm2_supported(type);
}

int gemm_kslices(int type, const WView & w, int64_t N, int64_t nbatch) {
    return gemm_uses_v2(type) ? gemm2_kslices(w, N, nbatch) : 1;
}

hipError_t launch_gemm(int type, const WView & w, const ActBuf & a, int64_t N, int64_t nbatch,
                       const GemmBatch & bt, float * dst, hipStream_t s, const KTime * kt) {
    if (gemm_uses_v2(type)) return launch_gemm2(type, w, a, N, nbatch, bt, dst, s, kt);
    const int64_t M = w.M, K = w.K;
    if (!a.dT || a.ldT < N * nbatch + 64 || K % 32 || M <= 0 || N <= 0 || nbatch <= 0 || a.K != K)
        return hipErrorInvalidValue;
    const bool kq = type == QMM_TYPE_Q4_K || type == QMM_TYPE_Q6_K || type == QMM_TYPE_IQ4_XS;
    if (kq && K % 256) return hipErrorInvalidValue;
    GemmParams p{};
    p.w = w;
    p.M = M;
    p.K = K;
    p.N = N;
    p.codes = a.codes;
    p.ldk = a.ldk;
    p.dT = a.dT;
    p.ldT = a.ldT;
    p.bt = bt;
    p.dst = dst;
    switch (type) {
        case QMM_TYPE_Q4_0:   return launch_t<QMM_TYPE_Q4_0, 2, 2>(p, nbatch, s, kt);
        case QMM_TYPE_Q8_0:   return launch_t<QMM_TYPE_Q8_0, 2, 2>(p, nbatch, s, kt);
        case QMM_TYPE_Q4_K:   return launch_t<QMM_TYPE_Q4_K, 2, 2>(p, nbatch, s, kt);
        case QMM_TYPE_Q6_K:   return launch_t<QMM_TYPE_Q6_K, 2, 2>(p, nbatch, s, kt);
        case QMM_TYPE_IQ4_XS: return launch_t<QMM_TYPE_IQ4_XS, 2, 2>(p, nbatch, s, kt);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
