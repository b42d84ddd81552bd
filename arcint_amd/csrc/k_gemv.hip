// k_gemv.hip - dequant-fused decode GEMV (N = 1..8 columns per task) on gfx950.
//
// Role of the reference's kernel_mul_mv_{q4_K,q6_K}_q8_1 (P01:3740-3921),
// kernel_mul_mv_q4_0_q8_1 (P02:6098-6220), kernel_mul_mv_iq4_xs_q8_1
// (P01:3457-3553), the Q8_0 matvec and the MUL_MAT_ID matvec
// (P01:3923-3964), redesigned for CDNA4 and for ggml-cpu's numerics instead
// of the reference's two-term q8_1 activations:
//  * lane r of a wave owns row r of a 64-row weight tile and walks groups of
//    256 weights along K; every weight load is one chunk plane of the tiled
//    image (one fully coalesced 1 KB wave load), and every lane decodes the
//    scales of a whole super-block (8 blocks of Q4_0/Q8_0) once;
//  * the activations are the vec_dot type's codes (q8_0 or q8_K, bit-exact
//    with ggml-cpu's from_float) from the pre-pass; a wave's group is the same
//    for all its lanes, so the codes, scales and sums are read with scalar
//    loads into SGPRs and feed v_dot4 as its scalar operand: no LDS, no
//    activation registers per lane.  The integer dot of every (sub-)block
//    equals ggml-cpu's exactly and only the fp32 combine order differs;
//  * W waves of a work-group split K and are added through LDS in a fixed
//    order; short matrices also split K over KS work-groups whose partial
//    sums are added to dst (zeroed by the pre-pass) with float atomics - no
//    device-scope fences, whose L2 write-backs would cost more than the whole
//    product;
//  * D stages of weight loads are in flight per wave in a register ring whose
//    loads are unconditional, so every wait is for a known load; a slot
//    refilled past the last stage reads a small L2-resident sink buffer
//    instead (re-reading real weights would go back to HBM: the weight loads
//    are non-temporal).
// A task is up to NC activation columns against one weight matrix; dense
// MUL_MAT derives tasks from the work-group index, MUL_MAT_ID reads
// device-built task lists.
#include "qmm_device.h"

#include <hip/hip_ext.h>

#include <algorithm>
#include <cstdlib>

namespace qmm {
namespace {

struct GemvParams {
    WView w;
    const int8_t * xc;           // activation codes [col][ldk]
    const float * xd;            // scales [col][ldk / BS]
    const int16_t * xs;          // code sums [col][ldk / SS]
    int64_t ldk;
    const GemvTask * tasks;      // list mode when non-null
    const int32_t * ntasks_dev;
    // dense mode: task -> batch b = task / tpb, columns (task % tpb) * NC ...
    int64_t ne11, ne12, r2, r3, ne02, tpb;
    int64_t d_nb1, d_nb2, d_nb3; // dst strides in floats
    float * dst;
    const uint8_t * sink;        // >= kSinkBytes of readable memory for loads past the end
    int W;                       // waves per work-group
    int KS;                      // work-groups per tile (K slices); > 1: atomics into zeroed dst
    int spw;                     // groups per wave
};

// wave-uniform (scalar) loads of the pre-quantized activations
typedef const __attribute__((address_space(4))) uint32_t cu32;
__device__ __forceinline__ uint32_t sld(const void * p, int i) { return ((cu32 *)p)[i]; }
__device__ __forceinline__ uint4 sld4(const void * p, int i) { return make_uint4(sld(p, i), sld(p, i + 1), sld(p, i + 2), sld(p, i + 3)); }
__device__ __forceinline__ float sldf(const void * p, int i) { return __builtin_bit_cast(float, sld(p, i)); }
// int16 number i of an int16 array (4-byte aligned)
__device__ __forceinline__ int slds16(const void * p, int i) { return (int)(int16_t)(sld(p, i >> 1) >> (16 * (i & 1))); }

// one group (256 weights) of the activation columns of a task
template <int NC>
struct XG {
    const int8_t * c[NC];        // codes of the group
    const float * d[NC];         // its scales
    const int16_t * s[NC];       // its code sums
};

__device__ __forceinline__ int dot16(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, const uint4 & a, int acc) {
    return dot4(w0, a.x, dot4(w1, a.y, dot4(w2, a.z, dot4(w3, a.w, acc))));
}

template <int TYPE> struct GV;

// ---- Q4_0: one stage per group: 8 code chunks (block p = chunk p) + d chunk
template <> struct GV<QMM_TYPE_Q4_0> {
    static constexpr int NST = 1, NL = 9, ND = 8, NS = 8;
    __device__ static void load(uint4 * r, const uint8_t * tg, int, int lane) {
        const uint8_t * p = tg + lane * 16;
#pragma unroll
        for (int c = 0; c < 9; ++c) r[c] = ld16_nt(p + c * kChunk);
    }
    template <int NC>
    __device__ static void dot(const uint4 * r, int, const XG<NC> & x, int nc, float * acc, int *) {
        const uint32_t dw2[4] = { r[8].x, r[8].y, r[8].z, r[8].w };
        const uint32_t m = 0x0F0F0F0Fu;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const uint4 q = r[p];
            const uint32_t l0 = q.x & m, l1 = q.y & m, l2 = q.z & m, l3 = q.w & m;
            const uint32_t h0 = (q.x >> 4) & m, h1 = (q.y >> 4) & m, h2 = (q.z >> 4) & m, h3 = (q.w >> 4) & m;
            const float dw = h2f(dw2[p >> 1] >> (16 * (p & 1)));
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                if (j < nc) {
                    int s = dot16(l0, l1, l2, l3, sld4(x.c[j], 8 * p), 0);
                    s = dot16(h0, h1, h2, h3, sld4(x.c[j], 8 * p + 4), s);
                    s -= 8 * slds16(x.s[j], p);                // codes are q, the weight is q - 8
                    acc[j] += (float)s * (dw * sldf(x.d[j], p));
                }
            }
        }
    }
};

// ---- Q8_0: two stages per group: blocks 4st..4st+3 (chunks 8st..8st+7) + d
template <> struct GV<QMM_TYPE_Q8_0> {
    static constexpr int NST = 2, NL = 9, ND = 8, NS = 8;
    __device__ static void load(uint4 * r, const uint8_t * tg, int st, int lane) {
        const uint8_t * p = tg + lane * 16;
#pragma unroll
        for (int c = 0; c < 8; ++c) r[c] = ld16_nt(p + (8 * st + c) * kChunk);
        r[8] = ld16(p + 16 * kChunk);                     // both stages: keep it cached
    }
    template <int NC>
    __device__ static void dot(const uint4 * r, int st, const XG<NC> & x, int nc, float * acc, int *) {
        const uint32_t dw2[4] = { r[8].x, r[8].y, r[8].z, r[8].w };
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
            const int p = 4 * st + pp;
            const uint4 q0 = r[2 * pp], q1 = r[2 * pp + 1];
            const uint32_t dsel = st ? dw2[2 + (pp >> 1)] : dw2[pp >> 1];
            const float dw = h2f(dsel >> (16 * (pp & 1)));
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                if (j < nc) {
                    int s = dot16(q0.x, q0.y, q0.z, q0.w, sld4(x.c[j], 8 * p), 0);
                    s = dot16(q1.x, q1.y, q1.z, q1.w, sld4(x.c[j], 8 * p + 4), s);
                    acc[j] += (float)s * (dw * sldf(x.d[j], p));
                }
            }
        }
    }
};

// ---- Q4_K: one stage per group: 8 code chunks + the header chunk ---------
// chunk c = qs[16c, 16c+16): low nibbles are weights 64(c/2) + 16(c%2) + i of
// sub-block 2(c/2), high nibbles the same + 32 of sub-block 2(c/2) + 1.
template <> struct GV<QMM_TYPE_Q4_K> {
    static constexpr int NST = 1, NL = 9, ND = 1, NS = 16;
    __device__ static void load(uint4 * r, const uint8_t * tg, int, int lane) {
        const uint8_t * p = tg + lane * 16;
#pragma unroll
        for (int c = 0; c < 9; ++c) r[c] = ld16_nt(p + c * kChunk);
    }
    template <int NC>
    __device__ static void dot(const uint4 * r, int, const XG<NC> & x, int nc, float * acc, int *) {
        const uint4 h = r[8];                              // d, dmin | scales[12]
        const float d = h2f(h.x), dmin = h2f(h.x >> 16);
        // 6-bit scales / mins (get_scale_min_k4, P01:2164-2176), one per byte
        const uint32_t sc03 = h.y & 0x3f3f3f3fu, mn03 = h.z & 0x3f3f3f3fu;
        const uint32_t sc47 = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
        const uint32_t mn47 = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
        int sc[8], mn[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sc[i] = (int)((sc03 >> (8 * i)) & 0xffu);
            sc[4 + i] = (int)((sc47 >> (8 * i)) & 0xffu);
            mn[i] = (int)((mn03 >> (8 * i)) & 0xffu);
            mn[4 + i] = (int)((mn47 >> (8 * i)) & 0xffu);
        }
        int isc[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) isc[j] = 0;
        const uint32_t m = 0x0F0F0F0Fu;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint4 q = r[c];
            const uint32_t l0 = q.x & m, l1 = q.y & m, l2 = q.z & m, l3 = q.w & m;
            const uint32_t h0 = (q.x >> 4) & m, h1 = (q.y >> 4) & m, h2 = (q.z >> 4) & m, h3 = (q.w >> 4) & m;
            const int jl = 2 * (c >> 1), xo = 16 * (c >> 1) + 4 * (c & 1);   // dwords
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                if (j < nc) {
                    const int sl = dot16(l0, l1, l2, l3, sld4(x.c[j], xo), 0);
                    const int sh = dot16(h0, h1, h2, h3, sld4(x.c[j], xo + 8), 0);
                    isc[j] += sc[jl] * sl + sc[jl + 1] * sh;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            if (j < nc) {
                int imn = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) imn += mn[i] * (slds16(x.s[j], 2 * i) + slds16(x.s[j], 2 * i + 1));
                acc[j] += sldf(x.d[j], 0) * (d * (float)isc[j] - dmin * (float)imn);
            }
        }
    }
};

// ---- Q6_K: two stages per group (half n = st) ------------------------------
// half n: ql chunks 4n..4n+3, qh chunks 8+2n, 9+2n, the scales chunk and d.
// Weight 128n + 32g + 16lh + i: ql chunk 4n + 2(g&1) + lh (low nibble for
// g < 2, high for g >= 2), qh chunk 2n + lh bits 2g..2g+1, scale and code
// sum index 8n + 2g + lh.
template <> struct GV<QMM_TYPE_Q6_K> {
    static constexpr int NST = 2, NL = 8, ND = 1, NS = 16;
    __device__ static void load(uint4 * r, const uint8_t * tg, int st, int lane) {
        const uint8_t * p = tg + lane * 16;
#pragma unroll
        for (int c = 0; c < 4; ++c) r[c] = ld16_nt(p + (4 * st + c) * kChunk);
        r[4] = ld16_nt(p + (8 + 2 * st) * kChunk);
        r[5] = ld16_nt(p + (9 + 2 * st) * kChunk);
        r[6] = ld16(p + 12 * kChunk);                      // both stages: keep it cached
        r[7].x = *reinterpret_cast<const uint16_t *>(tg + 13 * kChunk + lane * 2);
    }
    template <int NC>
    __device__ static void dot(const uint4 * r, int st, const XG<NC> & x, int nc, float * acc, int * isum) {
        if (st == 0) {
#pragma unroll
            for (int j = 0; j < NC; ++j) isum[j] = 0;
        }
        const uint32_t scw[4] = { r[6].x, r[6].y, r[6].z, r[6].w };
        const uint32_t m = 0x0F0F0F0Fu, m2 = 0x03030303u;
#pragma unroll
        for (int lh = 0; lh < 2; ++lh) {
            const uint4 qh = r[4 + lh];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint4 ql = r[lh + 2 * (g & 1)];
                const int sh = g < 2 ? 0 : 4;
                const uint32_t c0 = ((ql.x >> sh) & m) | (((qh.x >> (2 * g)) & m2) << 4);
                const uint32_t c1 = ((ql.y >> sh) & m) | (((qh.y >> (2 * g)) & m2) << 4);
                const uint32_t c2 = ((ql.z >> sh) & m) | (((qh.z >> (2 * g)) & m2) << 4);
                const uint32_t c3 = ((ql.w >> sh) & m) | (((qh.w >> (2 * g)) & m2) << 4);
                const int is = 8 * st + 2 * g + lh;
                const int sc = (int)(int8_t)((scw[is >> 2] >> (8 * (is & 3))) & 0xffu);
                const int xo = 32 * st + 8 * g + 4 * lh;         // dwords
#pragma unroll
                for (int j = 0; j < NC; ++j) {
                    if (j < nc) {
                        int s = dot16(c0, c1, c2, c3, sld4(x.c[j], xo), 0);
                        s -= 32 * slds16(x.s[j], is);           // codes are q, the weight q - 32
                        isum[j] += sc * s;
                    }
                }
            }
        }
        if (st == 1) {
            const float d = h2f(r[7].x);
#pragma unroll
            for (int j = 0; j < NC; ++j)
                if (j < nc) acc[j] += (d * sldf(x.d[j], 0)) * (float)isum[j];
        }
    }
};

// ---- IQ4_XS: one stage per group: 8 code chunks (sub-block ib = chunk ib)
// + the 8-byte header {d, scales_h, scales_l[4]} of the tail plane
template <> struct GV<QMM_TYPE_IQ4_XS> {
    static constexpr int NST = 1, NL = 9, ND = 1, NS = 16;
    __device__ static void load(uint4 * r, const uint8_t * tg, int, int lane) {
        const uint8_t * p = tg + lane * 16;
#pragma unroll
        for (int c = 0; c < 8; ++c) r[c] = ld16_nt(p + c * kChunk);
        const uint2 h = *reinterpret_cast<const uint2 *>(tg + 8 * kChunk + lane * 8);
        r[8].x = h.x;
        r[8].y = h.y;
    }
    template <int NC>
    __device__ static void dot(const uint4 * r, int, const XG<NC> & x, int nc, float * acc, int *) {
        const float dw = h2f(r[8].x);
        const uint32_t shi = r[8].x >> 16, slo = r[8].y;
        int isum[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) isum[j] = 0;
        const uint32_t m = 0x0F0F0F0Fu;
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            const uint4 q = r[ib];
            const int ls = (int)(((slo >> (4 * ib)) & 0xFu) | (((shi >> (2 * ib)) & 3u) << 4)) - 32;
            const uint32_t v0 = iq4_lookup(q.x & m), v1 = iq4_lookup(q.y & m), v2 = iq4_lookup(q.z & m), v3 = iq4_lookup(q.w & m);
            const uint32_t u0 = iq4_lookup((q.x >> 4) & m), u1 = iq4_lookup((q.y >> 4) & m);
            const uint32_t u2 = iq4_lookup((q.z >> 4) & m), u3 = iq4_lookup((q.w >> 4) & m);
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                if (j < nc) {
                    int s = dot16(v0, v1, v2, v3, sld4(x.c[j], 8 * ib), 0);
                    s = dot16(u0, u1, u2, u3, sld4(x.c[j], 8 * ib + 4), s);
                    isum[j] += ls * s;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < NC; ++j)
            if (j < nc) acc[j] += (dw * sldf(x.d[j], 0)) * (float)isum[j];
    }
};

// weight stages in flight per wave (register ring), by columns
// Stages in flight per wave.  One (the next stage is loaded once the current
// one is consumed; the other waves of the SIMD hide the latency) streams
// faster than deeper rings, whose many outstanding loads per wave queue up in
// the memory pipeline: 17408 x 5120 Q4_K 11.8 us at depth 1 against 13.4 us
// at depth 3.
template <int NC> constexpr int ring_depth() { return 1; }

// One work-group: W waves on one 64-row tile of one task's matrix and one of
// the tile's KS K slices; wave w takes groups [(ks W + w) spw, + spw).  Lane r
// owns row r.  At the end the W waves are added in LDS in a fixed order and
// wave 0 stores (KS == 1) or atomically adds (KS > 1) the row's sum.
template <int TYPE, int NC>
__global__ __launch_bounds__(512) void k_gemv(GemvParams p) {
    using T = GV<TYPE>;
    constexpr int NL = T::NL, NST = T::NST, ND = T::ND, NS = T::NS;
    constexpr int D = ring_depth<NC>();
    extern __shared__ __align__(16) float red[];       // [W][NC][64]
    __shared__ int64_t s_col[NC];      // activation column ids
    __shared__ int64_t s_doff[NC];     // float offset of dst row 0 per column

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // work-group -> (task, tile, K slice); these counts fit 32 bits
    const uint32_t ntl = (uint32_t)p.w.ntiles;
    const uint32_t ks = blockIdx.x % (uint32_t)p.KS, rest = blockIdx.x / (uint32_t)p.KS;
    const uint32_t tile = rest % ntl, task = rest / ntl;
    int mat, nc;
    if (p.tasks) {
        if (p.ntasks_dev && (int)task >= *p.ntasks_dev) return;     // uniform
        const GemvTask & t = p.tasks[task];
        mat = t.mat;
        nc = t.ncols < NC ? t.ncols : NC;
        if (tid < nc) {
            s_col[tid] = t.col[tid];
            s_doff[tid] = t.dst_off[tid];
        }
    } else {
        const uint32_t tpb = (uint32_t)p.tpb, ne12 = (uint32_t)p.ne12;
        const uint32_t b = task / tpb, tt = task - b * tpb;
        const uint32_t i3 = b / ne12, i2 = b - i3 * ne12;
        mat = (int)(i2 / (uint32_t)p.r2 + (i3 / (uint32_t)p.r3) * (uint32_t)p.ne02);
        const int64_t first = (int64_t)tt * NC;
        nc = (int)((p.ne11 - first) < NC ? (p.ne11 - first) : NC);
        if (tid < nc) {
            const int64_t i1 = first + tid;
            s_col[tid] = (int64_t)b * p.ne11 + i1;
            s_doff[tid] = i1 * p.d_nb1 + (int64_t)i2 * p.d_nb2 + (int64_t)i3 * p.d_nb3;
        }
    }
    if (mat < 0 || nc <= 0) return;    // uniform over the work-group
    __syncthreads();                   // s_col, s_doff
    nc = __builtin_amdgcn_readfirstlane(nc);

    const int G = (int)p.w.G;
    const int ga = ((int)ks * p.W + wave) * p.spw;                // this wave's groups [ga, gb)
    const int gb = ga + p.spw < G ? ga + p.spw : G;
    const int S = ga < gb ? (gb - ga) * NST : 0;                  // stages (uniform)
    const uint8_t * tbase = tile_group(p.w, mat, tile, 0);
    const size_t tgs = (size_t)p.w.tg;

    // per-column activation pointers at group 0 (uniform)
    const int8_t * xc0[NC];
    const float * xd0[NC];
    const int16_t * xs0[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int64_t col = j < nc ? s_col[j] : s_col[0];
        const int64_t cu = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(col >> 32)) << 32) |
                                     (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)col));
        xc0[j] = p.xc + cu * p.ldk;
        xd0[j] = p.xd + cu * (p.ldk / (256 / ND));
        xs0[j] = p.xs + cu * (p.ldk / (256 / NS));
    }

    float acc[NC];
    int st_state[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        acc[j] = 0.0f;
        st_state[j] = 0;
    }
    if (S > 0) {
        uint4 B[D][NL];
        auto load_stage = [&](uint4 * b, int s) {             // past the end: the sink
            const uint8_t * tg = s < S ? tbase + (size_t)(ga + s / NST) * tgs : p.sink;
            T::load(b, tg, s < S ? s % NST : 0, lane);
        };
#pragma unroll
        for (int i = 0; i < D; ++i) load_stage(B[i], i);
        for (int s = 0; s < S; s += D) {
#pragma unroll
            for (int i = 0; i < D; ++i) {
                if (s + i < S) {                                  // uniform
                    const int g = ga + (s + i) / NST;
                    XG<NC> x;
#pragma unroll
                    for (int j = 0; j < NC; ++j) {
                        x.c[j] = xc0[j] + (int64_t)g * 256;
                        x.d[j] = xd0[j] + (int64_t)g * ND;
                        x.s[j] = xs0[j] + (int64_t)g * NS;
                    }
                    T::template dot<NC>(B[i], (s + i) % NST, x, nc, acc, st_state);
                }
                load_stage(B[i], s + i + D);
            }
        }
    }

    // add the W waves in a fixed order
    const int64_t row = (int64_t)tile * kTileRows + lane;
    float tot[NC];
    if (p.W > 1) {
#pragma unroll
        for (int j = 0; j < NC; ++j) red[(wave * NC + j) * 64 + lane] = acc[j];
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            float v = red[j * 64 + lane];
            for (int w = 1; w < p.W; ++w) v += red[(w * NC + j) * 64 + lane];
            tot[j] = v;
        }
    } else {
#pragma unroll
        for (int j = 0; j < NC; ++j) tot[j] = acc[j];
    }
    if (row >= p.w.M) return;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        if (j < nc) {
            float * o = p.dst + s_doff[j] + row;
            if (p.KS == 1) *o = tot[j];
            else atomicAdd(o, tot[j]);
        }
    }
}

template <int TYPE>
hipError_t launch_t(const GemvParams & p, int nc, int64_t nwg, hipStream_t s, const KTime * kt) {
    const int threads = 64 * p.W;
    const size_t lds = p.W > 1 ? (size_t)p.W * nc * 64 * sizeof(float) : 0;
    switch (nc) {
#define QMM_NC(N)                                                                                  \
    case N:                                                                                        \
        if (kt) hipExtLaunchKernelGGL(k_gemv<TYPE, N>, dim3((unsigned)nwg), dim3(threads), (uint32_t)lds, s, \
                                      kt->start, kt->stop, 0, p);                                  \
        else k_gemv<TYPE, N><<<dim3((unsigned)nwg), threads, lds, s>>>(p);                         \
        break;
        QMM_NC(1) QMM_NC(2) QMM_NC(3) QMM_NC(4) QMM_NC(5) QMM_NC(6) QMM_NC(7) QMM_NC(8)
#undef QMM_NC
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

int env_int(const char * name, int dflt) {
    const char * e = getenv(name);
    return e ? atoi(e) : dflt;
}

}  // namespace

bool gemv_plan(int type, const WView & w, int nc, int64_t ntasks, bool allow_split, GemvPlan * pl) {
    if (!type_layout(type) || nc < 1 || nc > kMaxTaskCols || ntasks <= 0 || w.G <= 0 || w.ntiles <= 0) return false;
    pl->nc = nc;
    pl->ntasks = ntasks;
    // waves: about `target` in all (each with at least one group), at most
    // wmax per work-group; the rest of the split goes to work-groups per tile
    // (KS), which need dst zeroed before the launch
    const int64_t tiles = ntasks * w.ntiles;
    const int64_t target = std::max(1, env_int("QMM_GEMV_WAVES", 4096));
    // without split K (task lists: dst rows are not zeroed first) the K split
    // is all within the work-group, up to 8 waves
    const int64_t wmax = std::min(8, std::max(1, env_int("QMM_GEMV_WMAX", allow_split ? 1 : 8)));
    int64_t kw = std::min<int64_t>(w.G, std::max<int64_t>(1, (target + tiles - 1) / tiles));
    if (!allow_split) kw = std::min(kw, wmax);
    int64_t spw = (w.G + kw - 1) / kw;
    kw = (w.G + spw - 1) / spw;
    const int64_t W = std::min(kw, wmax);
    int64_t KS = allow_split ? (kw + W - 1) / W : 1;
    spw = (w.G + KS * W - 1) / (KS * W);
    KS = (w.G + spw * W - 1) / (spw * W);      // no work-group without groups
    pl->W = (int)W;
    pl->KS = (int)KS;
    pl->spw = (int)spw;
    const int64_t nwg = tiles * KS;
    return nwg > 0 && nwg < 0x7fffffff;
}

hipError_t launch_gemv(int type, const WView & w, const GemvPlan & pl, const ActBuf & a, const GemvTask * tasks,
                       const int32_t * ntasks_dev, const GemvDense * dense, float * dst, const void * sink,
                       hipStream_t s, const KTime * kt) {
    if (!sink || (!tasks && !dense) || pl.W < 1 || pl.W > 8 || pl.KS < 1 || pl.spw < 1 || a.ldk != w.G * 256 ||
        a.vdt != vec_dot_type(type))
        return hipErrorInvalidValue;
    GemvParams p{};
    p.w = w;
    p.xc = a.codes;
    p.xd = a.d;
    p.xs = a.sums;
    p.ldk = a.ldk;
    p.tasks = tasks;
    p.ntasks_dev = ntasks_dev;
    p.dst = dst;
    p.sink = (const uint8_t *)sink;
    p.W = pl.W;
    p.KS = pl.KS;
    p.spw = pl.spw;
    if (!tasks) {
        p.ne11 = dense->ne11;
        p.ne12 = dense->ne12;
        p.r2 = dense->r2;
        p.r3 = dense->r3;
        p.ne02 = dense->ne02;
        p.tpb = (dense->ne11 + pl.nc - 1) / pl.nc;
        p.d_nb1 = dense->d_nb1;
        p.d_nb2 = dense->d_nb2;
        p.d_nb3 = dense->d_nb3;
        if (p.tpb * dense->ne12 * dense->ne13 != pl.ntasks) return hipErrorInvalidValue;
    }
    const int64_t nwg = pl.ntasks * w.ntiles * pl.KS;
    switch (type) {
        case QMM_TYPE_Q4_0:   return launch_t<QMM_TYPE_Q4_0>(p, pl.nc, nwg, s, kt);
        case QMM_TYPE_Q8_0:   return launch_t<QMM_TYPE_Q8_0>(p, pl.nc, nwg, s, kt);
        case QMM_TYPE_Q4_K:   return launch_t<QMM_TYPE_Q4_K>(p, pl.nc, nwg, s, kt);
        case QMM_TYPE_Q6_K:   return launch_t<QMM_TYPE_Q6_K>(p, pl.nc, nwg, s, kt);
        case QMM_TYPE_IQ4_XS: return launch_t<QMM_TYPE_IQ4_XS>(p, pl.nc, nwg, s, kt);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
