// k_gemv.hip - dequant-fused decode GEMV (N = 1..8 columns per task) on gfx950.
//
// Role of the reference's kernel_mul_mv_{q4_K,q6_K}_q8_1 (P01:3740-3921),
// kernel_mul_mv_q4_0_q8_1 (P02:6098-6220), kernel_mul_mv_iq4_xs_q8_1
// (P01:3457-3553), mv_q45_K's Q5_K and mv_iq4_nl (P01:3736-3800,
// P01:3414-3455), the Q8_0 matvec and the MUL_MAT_ID matvec
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
//  * one stage of weight loads is in flight per wave (the v_dot4 kernels load
//    nothing past their last stage); the MFMA kernel's two-buffer ring loads
//    unconditionally, so every wait is for a known load, and a buffer refilled
//    past the last stage reads a small L2-resident sink buffer instead, all
//    lanes at one address (re-reading real weights would go back to HBM: the
//    weight loads are non-temporal).
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
    const int8_t * bsp;          // q8_K: split sub-block sums, 16 bytes at (super-block * ldT + col) * 16
    int64_t ldT;
    int64_t ldk;
    const GemvTask * tasks;      // list mode when non-null
    const int32_t * ntasks_dev;
    // dense mode: task -> batch b = task / tpb, columns (task % tpb) * NC ...
    int64_t ne11, ne12, r2, r3, ne02, tpb;
    int64_t d_nb1, d_nb2, d_nb3; // dst strides in floats
    float * dst;
    const uint8_t * sink;        // >= kSinkBytes of readable memory for loads past the end
    const uint8_t * base2;       // gate/up in one launch: the second image (dense: matrix 1; lists:
                                 // the task list runs twice, the second time on this stack), or null
    int64_t col_bs;              // dense mode: activation columns per batch
    int64_t up_doff;             // lists with base2: floats added to the second pass's dst offsets
    int glu;                     // lists with base2, >= 0: each work-group streams the gate tile (w)
                                 // and the up tile (base2) and stores act(gate) * up (enum qmm_glu)
    int W;                       // waves per work-group
    int KS;                      // work-groups per tile (K slices); > 1: atomics into zeroed dst
    int spw;                     // groups per wave
    int nct;                     // dense mode: columns per task
    int tw;                      // MFMA kernel: tiles per work-group (W / tw waves split K)
    int task0;                   // the grid is (KS, tiles or tile blocks, tasks from task0), blockIdx
                                 // is the position (launches of at most 65535 tasks each)
    int sh_mat;                  // lists: tasks of this matrix read the shared expert's images
    const uint8_t * sh_base;     // (its first image and, for base2's, its second); -1: none
    const uint8_t * sh_base2;
};

// tile-group 0 of (matrix, tile) of the first image, or (sec) of the second
__device__ __forceinline__ const uint8_t * mat_tile(const GemvParams & p, int mat, uint32_t tile, bool sec) {
    if (mat == p.sh_mat) {                                        // (uniform) the shared expert
        WView ws = p.w;
        ws.base = sec ? p.sh_base2 : p.sh_base;
        return tile_group(ws, 0, tile, 0);
    }
    if (sec) {
        WView w2 = p.w;
        w2.base = p.base2;
        return tile_group(w2, mat, tile, 0);
    }
    return tile_group(p.w, mat, tile, 0);
}

// wave-uniform (scalar) loads of the pre-quantized activations
typedef const __attribute__((address_space(4))) uint32_t cu32;
__device__ __forceinline__ uint32_t sld(const void * p, int i) { return ((cu32 *)p)[i]; }
__device__ __forceinline__ uint4 sld4(const void * p, int i) { return make_uint4(sld(p, i), sld(p, i + 1), sld(p, i + 2), sld(p, i + 3)); }
__device__ __forceinline__ float sldf(const void * p, int i) { return __builtin_bit_cast(float, sld(p, i)); }
// int16 number i of an int16 array (4-byte aligned)
__device__ __forceinline__ int slds16(const void * p, int i) { return (int)(int16_t)(sld(p, i >> 1) >> (16 * (i & 1))); }

// One group (256 weights) of the activation columns of a task, and how the stage dots read it:
// c4 = four code dwords from dword i, df = scale i, s16 = code sum i.  XG reads the pre-pass's
// codes in global memory with scalar loads (uniform over the wave); XL (the fused kernel) reads
// the wave's own quantization in LDS, a broadcast read.
template <int N>
struct XG {
    static constexpr int NC = N;
    const int8_t * c[N];         // codes of the group
    const float * d[N];          // its scales
    const int16_t * s[N];        // its code sums
    __device__ static uint4 c4(const int8_t * p, int i) { return sld4(p, i); }
    __device__ static float df(const float * p, int i) { return sldf(p, i); }
    __device__ static int s16(const int16_t * p, int i) { return slds16(p, i); }
};

__device__ __forceinline__ int dot16(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, const uint4 & a, int acc) {
    return dot4(w0, a.x, dot4(w1, a.y, dot4(w2, a.z, dot4(w3, a.w, acc))));
}

template <int TYPE> struct GV;

// ---- Q4_0: one stage per group: 8 code chunks (block p = chunk p) + d chunk
template <> struct GV<QMM_TYPE_Q4_0> {
    static constexpr int NST = 1, NL = 9, ND = 8, NS = 8;
    static constexpr int kReadEnd = 8 * kChunk + kTileRows * 16;         // chunks 0..8, 16 B a lane
    __device__ static void load(uint4 * r, const uint8_t * tg, int, int lane) {
        const uint8_t * p = tg + lane * 16;
#pragma unroll
        for (int c = 0; c < 9; ++c) r[c] = ld16_nt(p + c * kChunk);
    }
    template <class X>
    __device__ static void dot(const uint4 * r, int, const X & x, int nc, float * acc, int *) {
        constexpr int NC = X::NC;
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
                if (j < nc && !(QMM_RED == 3 && p == 7)) {      // (mutation 3: the group's last block dropped)
                    int s = dot16(l0, l1, l2, l3, X::c4(x.c[j], 8 * p), 0);
                    s = dot16(h0, h1, h2, h3, X::c4(x.c[j], 8 * p + 4), s);
                    s -= 8 * X::s16(x.s[j], p);                // codes are q, the weight is q - 8
                    acc[j] += (float)s * (dw * X::df(x.d[j], p));
                }
            }
        }
    }
};

// ---- Q8_0: two stages per group: blocks 4st..4st+3 (chunks 8st..8st+7) + d
template <> struct GV<QMM_TYPE_Q8_0> {
    static constexpr int NST = 2, NL = 9, ND = 8, NS = 8;
    static constexpr int kReadEnd = 16 * kChunk + kTileRows * 16;        // chunks 0..15 and 16
    __device__ static void load(uint4 * r, const uint8_t * tg, int st, int lane) {
        const uint8_t * p = tg + lane * 16;
#pragma unroll
        for (int c = 0; c < 8; ++c) r[c] = ld16_nt(p + (8 * st + c) * kChunk);
        r[8] = ld16(p + 16 * kChunk);                     // both stages: keep it cached
    }
    template <class X>
    __device__ static void dot(const uint4 * r, int st, const X & x, int nc, float * acc, int *) {
        constexpr int NC = X::NC;
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
                    int s = dot16(q0.x, q0.y, q0.z, q0.w, X::c4(x.c[j], 8 * p), 0);
                    s = dot16(q1.x, q1.y, q1.z, q1.w, X::c4(x.c[j], 8 * p + 4), s);
                    acc[j] += (float)s * (dw * X::df(x.d[j], p));
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
    static constexpr int kReadEnd = 8 * kChunk + kTileRows * 16;         // chunks 0..8
    __device__ static void load(uint4 * r, const uint8_t * tg, int, int lane) {
        const uint8_t * p = tg + lane * 16;
#pragma unroll
        for (int c = 0; c < 9; ++c) r[c] = ld16_nt(p + c * kChunk);
    }
    template <class X>
    __device__ static void dot(const uint4 * r, int, const X & x, int nc, float * acc, int *) {
        constexpr int NC = X::NC;
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
                    const int sl = dot16(l0, l1, l2, l3, X::c4(x.c[j], xo), 0);
                    const int sh = dot16(h0, h1, h2, h3, X::c4(x.c[j], xo + 8), 0);
                    isc[j] += sc[jl] * sl + sc[jl + 1] * sh;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            if (j < nc) {
                int imn = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) imn += mn[i] * (X::s16(x.s[j], 2 * i) + X::s16(x.s[j], 2 * i + 1));
                acc[j] += X::df(x.d[j], 0) * (d * (float)isc[j] - dmin * (float)imn);
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
    static constexpr int kReadEnd = 13 * kChunk + kTileRows * 2;         // chunks 0..12, then d (2 B a lane)
    __device__ static void load(uint4 * r, const uint8_t * tg, int st, int lane) {
        const uint8_t * p = tg + lane * 16;
#pragma unroll
        for (int c = 0; c < 4; ++c) r[c] = ld16_nt(p + (4 * st + c) * kChunk);
        r[4] = ld16_nt(p + (8 + 2 * st) * kChunk);
        r[5] = ld16_nt(p + (9 + 2 * st) * kChunk);
        r[6] = ld16(p + 12 * kChunk);                      // both stages: keep it cached
        r[7].x = *reinterpret_cast<const uint16_t *>(tg + 13 * kChunk + lane * 2);
    }
    template <class X>
    __device__ static void dot(const uint4 * r, int st, const X & x, int nc, float * acc, int * isum) {
        constexpr int NC = X::NC;
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
                        int s = dot16(c0, c1, c2, c3, X::c4(x.c[j], xo), 0);
                        s -= 32 * X::s16(x.s[j], is);           // codes are q, the weight q - 32
                        isum[j] += sc * s;
                    }
                }
            }
        }
        if (st == 1) {
            const float d = h2f(r[7].x);
#pragma unroll
            for (int j = 0; j < NC; ++j)
                if (j < nc) acc[j] += (d * X::df(x.d[j], 0)) * (float)isum[j];
        }
    }
};

// ---- IQ4_XS: one stage per group: 8 code chunks (sub-block ib = chunk ib)
// + the 8-byte header {d, scales_h, scales_l[4]} of the tail plane
template <> struct GV<QMM_TYPE_IQ4_XS> {
    static constexpr int NST = 1, NL = 9, ND = 1, NS = 16;
    static constexpr int kReadEnd = 8 * kChunk + kTileRows * 8;          // chunks 0..7, then the 8 B header
    __device__ static void load(uint4 * r, const uint8_t * tg, int, int lane) {
        const uint8_t * p = tg + lane * 16;
#pragma unroll
        for (int c = 0; c < 8; ++c) r[c] = ld16_nt(p + c * kChunk);
        const uint2 h = *reinterpret_cast<const uint2 *>(tg + 8 * kChunk + lane * 8);
        r[8].x = h.x;
        r[8].y = h.y;
    }
    template <class X>
    __device__ static void dot(const uint4 * r, int, const X & x, int nc, float * acc, int *) {
        constexpr int NC = X::NC;
        const float dw = h2f(r[8].x);
        const uint32_t shi = r[8].x >> 16, slo = r[8].y;
        int isum[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) isum[j] = 0;
        const Iq4Regs kr = iq4_regs();
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            const uint4 q = r[ib];
            const int ls = (int)(((slo >> (4 * ib)) & 0xFu) | (((shi >> (2 * ib)) & 3u) << 4)) - 32;
            uint32_t v0, v1, v2, v3, u0, u1, u2, u3;
            iq4_lookup8(q.x, kr, v0, u0); iq4_lookup8(q.y, kr, v1, u1);
            iq4_lookup8(q.z, kr, v2, u2); iq4_lookup8(q.w, kr, v3, u3);
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                if (j < nc) {
                    int s = dot16(v0, v1, v2, v3, X::c4(x.c[j], 8 * ib), 0);
                    s = dot16(u0, u1, u2, u3, X::c4(x.c[j], 8 * ib + 4), s);
                    isum[j] += ls * s;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < NC; ++j)
            if (j < nc) acc[j] += (dw * X::df(x.d[j], 0)) * (float)isum[j];
    }
};

// ---- IQ4_NL: Q4_0's stage (8 code chunks + the d chunk), the codes through the codebook
template <> struct GV<QMM_TYPE_IQ4_NL> {
    static constexpr int NST = 1, NL = 9, ND = 8, NS = 8;
    static constexpr int kReadEnd = GV<QMM_TYPE_Q4_0>::kReadEnd;
    __device__ static void load(uint4 * r, const uint8_t * tg, int st, int lane) { GV<QMM_TYPE_Q4_0>::load(r, tg, st, lane); }
    template <class X>
    __device__ static void dot(const uint4 * r, int, const X & x, int nc, float * acc, int *) {
        constexpr int NC = X::NC;
        const uint32_t dw2[4] = { r[8].x, r[8].y, r[8].z, r[8].w };
        const Iq4Regs kr = iq4_regs();
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const uint4 q = r[p];
            uint32_t v0, v1, v2, v3, u0, u1, u2, u3;
            iq4_lookup8(q.x, kr, v0, u0); iq4_lookup8(q.y, kr, v1, u1);
            iq4_lookup8(q.z, kr, v2, u2); iq4_lookup8(q.w, kr, v3, u3);
            const float dw = h2f(dw2[p >> 1] >> (16 * (p & 1)));
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                if (j < nc) {
                    int s = dot16(v0, v1, v2, v3, X::c4(x.c[j], 8 * p), 0);
                    s = dot16(u0, u1, u2, u3, X::c4(x.c[j], 8 * p + 4), s);
                    acc[j] += (float)s * (dw * X::df(x.d[j], p));
                }
            }
        }
    }
};

// ---- Q5_K: Q4_K's stage plus the two qh chunks: byte i of qh chunk 9 + h holds the fifth bits
// of position 16 h + i of all four 64-weight chunks (bit 2 cc low nibble, 2 cc + 1 high)
template <> struct GV<QMM_TYPE_Q5_K> {
    static constexpr int NST = 1, NL = 11, ND = 1, NS = 16;
    static constexpr int kReadEnd = 10 * kChunk + kTileRows * 16;        // chunks 0..10
    __device__ static void load(uint4 * r, const uint8_t * tg, int, int lane) {
        const uint8_t * p = tg + lane * 16;
#pragma unroll
        for (int c = 0; c < 11; ++c) r[c] = ld16_nt(p + c * kChunk);
    }
    template <class X>
    __device__ static void dot(const uint4 * r, int, const X & x, int nc, float * acc, int *) {
        constexpr int NC = X::NC;
        const uint4 h = r[8];                              // d, dmin | scales[12]
        const float d = h2f(h.x), dmin = h2f(h.x >> 16);
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
        const uint32_t m = 0x0F0F0F0Fu, b1 = 0x01010101u;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint4 q = r[c], qh = r[9 + (c & 1)];
            const int bl = 2 * (c >> 1), bh = bl + 1;            // fifth-bit positions
            const uint32_t l0 = (q.x & m) | (((qh.x >> bl) & b1) << 4), l1 = (q.y & m) | (((qh.y >> bl) & b1) << 4);
            const uint32_t l2 = (q.z & m) | (((qh.z >> bl) & b1) << 4), l3 = (q.w & m) | (((qh.w >> bl) & b1) << 4);
            const uint32_t h0 = ((q.x >> 4) & m) | (((qh.x >> bh) & b1) << 4), h1 = ((q.y >> 4) & m) | (((qh.y >> bh) & b1) << 4);
            const uint32_t h2 = ((q.z >> 4) & m) | (((qh.z >> bh) & b1) << 4), h3 = ((q.w >> 4) & m) | (((qh.w >> bh) & b1) << 4);
            const int jl = 2 * (c >> 1), xo = 16 * (c >> 1) + 4 * (c & 1);   // dwords
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                if (j < nc) {
                    const int sl = dot16(l0, l1, l2, l3, X::c4(x.c[j], xo), 0);
                    const int sh = dot16(h0, h1, h2, h3, X::c4(x.c[j], xo + 8), 0);
                    isc[j] += sc[jl] * sl + sc[jl + 1] * sh;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            if (j < nc) {
                int imn = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) imn += mn[i] * (X::s16(x.s[j], 2 * i) + X::s16(x.s[j], 2 * i + 1));
                acc[j] += X::df(x.d[j], 0) * (d * (float)isc[j] - dmin * (float)imn);
            }
        }
    }
};

// weight stages in flight per wave (register ring), by columns
// Stages in flight per wave.  One (the next stage is loaded once the current
// one is consumed; the other waves of the SIMD hide the latency) streams
// faster than deeper rings, whose many outstanding loads per wave queue up in
// the memory pipeline: 17408 x 5120 Q4_K 11.8 us at depth 1 against 13.4 us
// at depth 3.
template <int NC> constexpr int ring_depth() { return 1; }

// ---- index math of the two GEMV kernels, shared with the host replay of their loads --------
// (gemv_extent below walks every work-group, wave and stage of a plan with these functions)
// work-group b of a launch of n units (tiles or tile blocks) per task and KS K slices
struct WgPos { uint32_t ks, unit, task; };
__host__ __device__ __forceinline__ WgPos wg_pos(uint32_t b, uint32_t KS, uint32_t n) {
    const uint32_t rest = b / KS;
    return WgPos{ b % KS, rest % n, rest / n };
}
// dense task -> batch b = i2 + i3 ne12, column tile tt of the batch, and the weight matrix
struct DenseTask { uint32_t b, tt, i2, i3; int mat; };
__host__ __device__ __forceinline__ DenseTask dense_task(uint32_t task, uint32_t tpb, uint32_t ne12, uint32_t r2,
                                                         uint32_t r3, uint32_t ne02) {
    DenseTask d;
    d.b = task / tpb;
    d.tt = task - d.b * tpb;
    d.i3 = d.b / ne12;
    d.i2 = d.b - d.i3 * ne12;
    d.mat = (int)(d.i2 / r2 + (d.i3 / r3) * ne02);
    return d;
}
// v_dot4 kernel: wave `wave` of K slice ks streams S stages from group ga on (S = 0: none)
__host__ __device__ __forceinline__ void dot4_stages(int ks, int W, int wave, int spw, int G, int nst, int & ga, int & S) {
    ga = (ks * W + wave) * spw;
    const int gb = ga + spw < G ? ga + spw : G;
    S = ga < gb ? (gb - ga) * nst : 0;
}
// MFMA kernel: the work-group of K slice ks stages the activations of groups [gw, gw + ngw); its
// K wave kw streams groups [ga, ga + nsw)
__host__ __device__ __forceinline__ void mma_groups(int ks, int WK, int kw, int spw, int G, int & gw, int & ngw, int & ga,
                                                    int & nsw) {
    gw = ks * WK * spw;
    ngw = gw + WK * spw < G ? WK * spw : G - gw;
    ga = gw + kw * spw;
    nsw = ga >= G ? 0 : (ga + spw < G ? spw : G - ga);
}
// the group whose tile-group stage s of a wave starting at group ga loads (s < S)
__host__ __device__ __forceinline__ int stage_group(int ga, int s, int nst) { return ga + s / nst; }

// One work-group: W waves on one 64-row tile of one task's matrix and one of
// the tile's KS K slices; wave w takes groups [(ks W + w) spw, + spw).  Lane r
// owns row r.  At the end the W waves are added in LDS in a fixed order and
// wave 0 stores (KS == 1) or atomically adds (KS > 1) the row's sum.
template <int TYPE, int NC>
__global__ __launch_bounds__(512) void k_gemv(GemvParams p) {
    using T = GV<TYPE>;
    constexpr int NL = T::NL, NST = T::NST, ND = T::ND, NS = T::NS;
    constexpr int D = ring_depth<NC>();
    static_assert(NC <= kMaxTaskCols, "a task holds kMaxTaskCols columns");
    extern __shared__ __align__(16) float red[];       // [W][NC][64]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // work-group -> (task, tile, K slice); these counts fit 32 bits
    static_assert(T::kReadEnd <= tile_group_bytes(TYPE) && tile_group_bytes(TYPE) <= (int)kSinkBytes,
                  "a stage reads inside one tile-group, which fits in the sink");
    // the grid's dimensions are the position (work-group ks + KS (tile + ntl task) of wg_pos's
    // numbering): no divisions and no branch ahead of the first weight load
    const uint32_t ks = blockIdx.x, tile = blockIdx.y, task = blockIdx.z + (uint32_t)p.task0;
    int mat, nc;
    bool sec = false;                  // the second image (gate/up in one launch)
    // per column: activation column id and float offset of dst row 0, uniform
    // registers (no LDS copy and barrier ahead of the first weight load)
    int64_t colv[NC], doffv[NC];
    if (p.tasks) {
        const int ntk = p.ntasks_dev ? *p.ntasks_dev : 0x7fffffff;   // one load of the task count
        uint32_t tk = task;
        if (p.base2 && p.glu < 0 && (int)tk >= ntk) {             // the second pass over the list
            tk -= (uint32_t)ntk;
            sec = true;
        }
        if ((int)tk >= ntk) return;                               // uniform
        const GemvTask & t = p.tasks[tk];
        const int64_t dadd = sec ? p.up_doff : 0;
        mat = t.mat;
        nc = t.ncols < NC ? t.ncols : NC;
        if (mat < 0) {                                            // pairs of invalid ids: zero rows
            const int64_t row = (int64_t)tile * kTileRows + lane;
            if (ks == 0 && wave == 0 && row < p.w.M)
                for (int j = 0; j < nc; ++j) p.dst[t.c[j].dst_off + dadd + row] = 0.0f;
            return;                                               // uniform
        }
#pragma unroll
        for (int j = 0; j < NC; ++j) {                            // c[] holds kMaxTaskCols >= NC
            colv[j] = j < nc ? t.c[j].col : t.c[0].col;
            doffv[j] = (j < nc ? t.c[j].dst_off : 0) + dadd;
        }
    } else {
        // (task 0 is batch 0, column tile 0 and matrix 0 whatever the divisors: the one task of a
        // single-batch decode product takes no divisions)
        const DenseTask dt = task == 0 ? DenseTask{ 0, 0, 0, 0, 0 }
                                       : dense_task(task, (uint32_t)p.tpb, (uint32_t)p.ne12, (uint32_t)p.r2,
                                                    (uint32_t)p.r3, (uint32_t)p.ne02);
        mat = dt.mat;
        if (p.base2 && mat == 1) {                                // gate/up in one launch
            mat = 0;
            sec = true;
        }
        const int64_t first = (int64_t)dt.tt * NC;
        nc = (int)((p.ne11 - first) < NC ? (p.ne11 - first) : NC);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int64_t i1 = first + (j < nc ? j : 0);
            colv[j] = (int64_t)dt.b * p.col_bs + i1;
            doffv[j] = i1 * p.d_nb1 + (int64_t)dt.i2 * p.d_nb2 + (int64_t)dt.i3 * p.d_nb3;
        }
    }
    if (mat < 0 || nc <= 0) return;    // uniform over the work-group
    nc = __builtin_amdgcn_readfirstlane(nc);

    const int G = (int)p.w.G;
    int ga, S;                                                    // this wave's first group, its stages (uniform)
    dot4_stages((int)ks, p.W, wave, p.spw, G, NST, ga, S);
    const uint8_t * tbase = mat_tile(p, mat, tile, sec);
    const size_t tgs = (size_t)p.w.tg;

    // per-column activation pointers at group 0 (uniform)
    const int8_t * xc0[NC];
    const float * xd0[NC];
    const int16_t * xs0[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int64_t col = colv[j];
        const int64_t cu = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(col >> 32)) << 32) |
                                     (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)col));
        xc0[j] = p.xc + cu * p.ldk;
        xd0[j] = p.xd + cu * (p.ldk / (256 / ND));
        xs0[j] = p.xs + cu * (p.ldk / (256 / NS));
    }

    float acc[NC], accu[NC];
    int st_state[NC];
    // the wave's groups of one image into a[] (gate/up with GLU: the gate tile, then the up tile)
    auto stream = [&](const uint8_t * tb, float (&a)[NC]) {
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            a[j] = 0.0f;
            st_state[j] = 0;
        }
        if (S <= 0) return;
        uint4 B[D][NL];
        auto load_stage = [&](uint4 * b, int s) {             // past the end: the sink
            const uint8_t * tg = s < S ? tb + (size_t)stage_group(ga, s, NST) * tgs : p.sink;
            T::load(b, tg, s < S ? s % NST : 0, lane);
        };
#pragma unroll
        for (int i = 0; i < D; ++i) load_stage(B[i], i);
        for (int s = 0; s < S; s += D) {
#pragma unroll
            for (int i = 0; i < D; ++i) {
                if (s + i < S) {                                  // uniform
                    const int g = stage_group(ga, s + i, NST);
                    XG<NC> x;
#pragma unroll
                    for (int j = 0; j < NC; ++j) {
                        x.c[j] = xc0[j] + (int64_t)g * 256;
                        x.d[j] = xd0[j] + (int64_t)g * ND;
                        x.s[j] = xs0[j] + (int64_t)g * NS;
                    }
                    T::dot(B[i], (s + i) % NST, x, nc, a, st_state);
                }
                // (no stage past the last: with one stage in flight nothing else is outstanding
                // here, and 5440 waves re-reading one stage of the sink at their end cost the
                // chip ~50 MB of L2 reads at once)
                if (s + i + D < S) load_stage(B[i], s + i + D);
            }
        }
    };
    const bool glu = p.glu >= 0;                                  // uniform (lists only)
    stream(tbase, acc);
    if (glu) stream(mat_tile(p, mat, tile, true), accu);

    // add the W waves in a fixed order (with the GLU: both sums, then act(gate) * up)
    const int64_t row = (int64_t)tile * kTileRows + lane;
    float tot[NC];
    if (p.W > 1) {
        const int NV = glu ? 2 * NC : NC;
#pragma unroll
        for (int j = 0; j < NC; ++j) red[(wave * NV + j) * 64 + lane] = acc[j];
        if (glu) {
#pragma unroll
            for (int j = 0; j < NC; ++j) red[(wave * NV + NC + j) * 64 + lane] = accu[j];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            float v = red[j * 64 + lane];
            for (int w = 1; w < p.W; ++w) v += red[(w * NV + j) * 64 + lane];
            if (glu) {
                float u = red[(NC + j) * 64 + lane];
                for (int w = 1; w < p.W; ++w) u += red[(w * NV + NC + j) * 64 + lane];
                v = glu_apply(p.glu, v, u);
            }
            tot[j] = v;
        }
    } else {
#pragma unroll
        for (int j = 0; j < NC; ++j) tot[j] = glu ? glu_apply(p.glu, acc[j], accu[j]) : acc[j];
    }
    if (row >= p.w.M) return;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        if (j < nc) {
            float * o = p.dst + doffv[j] + row;
            if (p.KS == 1) *o = tot[j];
            else atomicAdd(o, tot[j]);
        }
    }
}

// ---- few columns (3..8) on v_mfma_i32_32x32x32_i8 ---------------------------
// A work-group is W waves on W consecutive 64-row tiles of one task's matrix
// over one of KS K slices (KS > 1: atomics into zeroed dst).  The slice's
// activation codes of the task's columns are staged once in LDS and shared by
// the W waves; the weight stream is the same tiled image as k_gemv's (lane =
// row), one stage ahead of the compute.  The dots run on the MFMA:
// A = the task's activation columns (lane l: column l % 32, zeros past nc; k
// half l / 32), B = two MFMAs per 32 weights, rows 0-31 and 32-63 of the tile.
// A lane loads its own row's weights; v_permlane32_swap trades lanes 32-63 of
// the lanes' k 0-15 for lanes 0-31 of their k 16-31, which is exactly the B
// layout of rows 0-31 (first result) and of rows 32-63 (second).  Per-row
// scales are applied after the MFMA on the integer results (Q4_K, IQ4_XS) or
// in the float epilogue (Q4_0, Q8_0), swapped to the output lanes the same
// way.  The output lane holds row l % 32 for columns 4 (l / 32) + r in
// registers r < 4.  At N = 8 this is about a third of the VALU work of eight
// v_dot4 per 32 weights and column.
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ void swap_halves(const uint4 & x, const uint4 & y, v4i & op0, v4i & op1) {
    const auto a = __builtin_amdgcn_permlane32_swap(x.x, y.x, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(x.y, y.y, false, false);
    const auto c = __builtin_amdgcn_permlane32_swap(x.z, y.z, false, false);
    const auto d = __builtin_amdgcn_permlane32_swap(x.w, y.w, false, false);
    op0 = v4i{ (int)a[0], (int)b[0], (int)c[0], (int)d[0] };
    op1 = v4i{ (int)a[1], (int)b[1], (int)c[1], (int)d[1] };
}
// a per-row value: rows 0-31 (r0) and rows 32-63 (r1) in the output lanes (row = lane % 32)
__device__ __forceinline__ void swap_rows(uint32_t v, uint32_t & r0, uint32_t & r1) {
    const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    r0 = a[0];
    r1 = a[1];
}
__device__ __forceinline__ uint4 map4(const uint4 & q, uint32_t (*f)(uint32_t)) { return make_uint4(f(q.x), f(q.y), f(q.z), f(q.w)); }
// the 32 codes of q through the codebook (iq4_lookup8): lo from the low nibbles, hi from the high
__device__ __forceinline__ void iq4_map8(const uint4 & q, const Iq4Regs & k, uint4 & lo, uint4 & hi) {
    iq4_lookup8(q.x, k, lo.x, hi.x); iq4_lookup8(q.y, k, lo.y, hi.y);
    iq4_lookup8(q.z, k, lo.z, hi.z); iq4_lookup8(q.w, k, lo.w, hi.w);
}
__device__ __forceinline__ uint4 nib(const uint4 & q, int sh) {
    const uint32_t m = 0x0F0F0F0Fu;
    return make_uint4((q.x >> sh) & m, (q.y >> sh) & m, (q.z >> sh) & m, (q.w >> sh) & m);
}

// Accumulators of the output lane.  A task has up to CM columns (8, 16 or 32: the MFMA's A
// operand holds 32); NR = CM / 2 registers of each 32-row MFMA result carry them: register r
// of lane l is column 8 (r / 4) + 4 (l / 32) + r % 4 of row l % 32.  Element NR t + r of the
// accumulator is register r of row tile t (rows 32 t + l % 32).  Each consume step ends with
// an empty asm on the whole vector: otherwise the compiler sinks every block's consumption
// below all the MFMAs and keeps their 16-register results live.
template <int N> using vNi = int __attribute__((ext_vector_type(N)));
template <int N> using vNf = float __attribute__((ext_vector_type(N)));

// column of accumulator register r (of a row tile) for lane half h
__host__ __device__ constexpr int mma_col(int r, int h) { return 8 * (r / 4) + 4 * h + (r & 3); }

// acc[NR t + r] += s_t * e_t[r]; the products fit 24 bits (full-rate multiplies)
template <int NR>
__device__ __forceinline__ void scale_add(const v16i & e0, const v16i & e1, int s0, int s1, vNi<2 * NR> & acc) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        acc[r] += __mul24(s0, e0[r]);
        acc[NR + r] += __mul24(s1, e1[r]);
    }
    asm volatile("" : "+v"(acc));
}
// out[NR t + r] += (i * dw_t) * dx[r] with i read from the magic-biased result e_t[r]: the bits
// of 12582912 + i, so fma(bits as float, dw, -12582912 dw) is i dw rounded once
template <int NR>
__device__ __forceinline__ void bf_epilogue(const v16i & e0, const v16i & e1, float dw0, float dw1, const float (&dx)[NR],
                                            vNf<2 * NR> & out) {
    const float nm0 = -12582912.0f * dw0, nm1 = -12582912.0f * (QMM_RED == 4 ? dw0 : dw1);   // (mutation 4)
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int i0 = e0[r], i1 = e1[r];
        out[r] = __builtin_fmaf(__builtin_fmaf(__builtin_bit_cast(float, i0), dw0, nm0), dx[r], out[r]);
        out[NR + r] = __builtin_fmaf(__builtin_fmaf(__builtin_bit_cast(float, i1), dw1, nm1), dx[r], out[NR + r]);
    }
    asm volatile("" : "+v"(out));
}

// One stage of the MFMA GEMV on the weights rw of the lane's row: A operands from the LDS
// codes at xag (block b at 32 b), the scales of the lane's output columns at xdg (CM floats
// per block, the lane's first at + 4 h), Q4_K split sums at xsg (bh[8], bl[8] of the lane's
// column).  A scheduling barrier per block bounds the live MFMA results: the K-quants issue
// block j's MFMAs before they consume block j - 1's, Q4_0 / Q8_0 / IQ4_NL (whose magic
// accumulator input takes 16 more registers) consume each block's in its own group.
// Q6_K (two stages per group, `iacc` carrying the super-block's integer sum across them):
// block g of half st is 32 weights whose k halves (lane halves after the swap) have their own
// int8 scales, so each takes its own MFMA with the other half's operand zero.
template <int TYPE, int CM, int NL>
__device__ __forceinline__ void mma_stage(const uint4 (&rw)[NL], int st, const uint8_t * xag, const float * xdg,
                                          const uint8_t * xsg, int h, const v16i & magic, vNf<CM> & out,
                                          vNi<CM> & iacc) {
    constexpr int NR = CM / 2;
    constexpr bool KQ = TYPE == QMM_TYPE_Q4_K, IQ = TYPE == QMM_TYPE_IQ4_XS, Q8 = TYPE == QMM_TYPE_Q8_0;
    constexpr bool NLQ = TYPE == QMM_TYPE_IQ4_NL;                // Q4_0's blocks through the codebook
    constexpr bool Q6 = TYPE == QMM_TYPE_Q6_K;
    constexpr bool BF = TYPE == QMM_TYPE_Q4_0 || Q8 || NLQ;
    constexpr bool HALVES = Q8 || Q6;                             // a group takes two stages
    constexpr int NB = Q8 ? 4 : 8;                                // 32-weight blocks per stage
    auto a_op = [&](int b) -> v4i { return *reinterpret_cast<const v4i *>(xag + 32 * (HALVES ? 4 * st + b : b)); };
    // the lane's NR column scales of block b: quads at columns 8 q + 4 h
    auto dx_op = [&](int b, float (&d)[NR]) {
        const float * x = xdg + (Q8 ? 4 * st + b : b) * CM;
#pragma unroll
        for (int q = 0; q < NR / 4; ++q) {
            const float4 v = *reinterpret_cast<const float4 *>(x + 8 * q);
            d[4 * q] = v.x; d[4 * q + 1] = v.y; d[4 * q + 2] = v.z; d[4 * q + 3] = v.w;
        }
    };
    if constexpr (BF) {
        const uint32_t dw2[4] = { rw[8].x, rw[8].y, rw[8].z, rw[8].w };
        const Iq4Regs kr = iq4_regs();                        // IQ4_NL: the codebook in VGPRs
        v4i an = a_op(0);                                     // LDS reads one block ahead
        float dn[NR];
        dx_op(0, dn);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int blk = Q8 ? 4 * st + b : b;                  // block of the group
            uint32_t d0b, d1b;
            swap_rows((dw2[blk >> 1] >> (16 * (blk & 1))) & 0xffffu, d0b, d1b);
            const float dw0 = h2f(d0b), dw1 = h2f(d1b);
            uint4 lo, hi;
            if constexpr (Q8) {
                lo = rw[2 * b];
                hi = rw[2 * b + 1];
            } else if constexpr (NLQ) {
                iq4_map8(rw[b], kr, lo, hi);
            } else {
                lo = map4(nib(rw[b], 0), q4_minus8);
                hi = map4(nib(rw[b], 4), q4_minus8);
            }
            v4i op0, op1;
            swap_halves(lo, hi, op0, op1);
            const v4i av = an;
            float dxb[NR];
#pragma unroll
            for (int r = 0; r < NR; ++r) dxb[r] = dn[r];
            if (b + 1 < NB) {
                an = a_op(b + 1);
                dx_op(b + 1, dn);
            }
            const v16i e0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, op0, magic, 0, 0, 0);
            const v16i e1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, op1, magic, 0, 0, 0);
            bf_epilogue<NR>(e0, e1, dw0, dw1, dxb, out);      // consumed in its own block: the
            __builtin_amdgcn_sched_barrier(0);                // SIMD's other waves cover the latency
        }
    } else if constexpr (KQ) {
        // sub-block j: one MFMA per 32 rows on the raw nibbles, its 6-bit scale applied per
        // row on the integer result; the min term sum_j m_j (64 bh_j + bl_j) is two MFMAs with
        // A = bh (then bl) of the lane's column at k = j and B = the row's mins
        const uint4 hd = rw[8];                               // d, dmin | scales[12]
        const uint32_t sc03 = hd.y & 0x3f3f3f3fu, mn03 = hd.z & 0x3f3f3f3fu;
        const uint32_t sc47 = (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u);
        const uint32_t mn47 = ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u);
        uint32_t scw[2][2], mnw[2][2];                        // [word][tile]
        swap_rows(sc03, scw[0][0], scw[0][1]);
        swap_rows(sc47, scw[1][0], scw[1][1]);
        swap_rows(mn03, mnw[0][0], mnw[0][1]);
        swap_rows(mn47, mnw[1][0], mnw[1][1]);
        vNi<CM> isc = {};
        v16i pe0, pe1;
        int ps0 = 0, ps1 = 0;
        v4i an = a_op(0);                                     // LDS reads one block ahead
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint4 lq = nib(rw[2 * (j >> 1)], 4 * (j & 1)), hq = nib(rw[2 * (j >> 1) + 1], 4 * (j & 1));
            v4i op0, op1;
            swap_halves(lq, hq, op0, op1);
            const v4i av = an;
            if (j + 1 < 8) an = a_op(j + 1);
            const v16i e0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, op0, v16i{}, 0, 0, 0);
            const v16i e1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, op1, v16i{}, 0, 0, 0);
            if (j > 0) scale_add<NR>(pe0, pe1, ps0, ps1, isc);
            __builtin_amdgcn_sched_barrier(0);
            pe0 = e0;
            pe1 = e1;
            ps0 = (int)((scw[j >> 2][0] >> (8 * (j & 3))) & 0xffu);
            ps1 = (int)((scw[j >> 2][1] >> (8 * (j & 3))) & 0xffu);
        }
        scale_add<NR>(pe0, pe1, ps0, ps1, isc);
        const uint4 sp = *reinterpret_cast<const uint4 *>(xsg);   // zeros for lanes without a column
        const v4i ah = h ? v4i{} : v4i{ (int)sp.x, (int)sp.y, 0, 0 };
        const v4i al = h ? v4i{} : v4i{ (int)sp.z, (int)sp.w, 0, 0 };
        const v4i bm0 = h ? v4i{} : v4i{ (int)mnw[0][0], (int)mnw[1][0], 0, 0 };
        const v4i bm1 = h ? v4i{} : v4i{ (int)mnw[0][1], (int)mnw[1][1], 0, 0 };
        const v16i mh0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, bm0, v16i{}, 0, 0, 0);
        const v16i ml0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, bm0, v16i{}, 0, 0, 0);
        const v16i mh1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, bm1, v16i{}, 0, 0, 0);
        const v16i ml1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, bm1, v16i{}, 0, 0, 0);
        float dx0[NR];
        dx_op(0, dx0);
        uint32_t dd0, dd1, dm0, dm1;
        swap_rows(hd.x & 0xffffu, dd0, dd1);
        swap_rows(hd.x >> 16, dm0, dm1);
        const float d[2] = { h2f(dd0), h2f(dd1) }, dmin[2] = { h2f(dm0), h2f(dm1) };
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int imn0 = 64 * mh0[r] + ml0[r], imn1 = 64 * mh1[r] + ml1[r];
            out[r] += dx0[r] * (d[0] * (float)isc[r] - dmin[0] * (float)imn0);
            out[NR + r] += dx0[r] * (d[1] * (float)isc[NR + r] - dmin[1] * (float)imn1);
        }
    } else if constexpr (Q6) {
        // half st: ql chunks rw[0..3] (4 st + c), qh rw[4], rw[5] (lh = 0, 1), the 16 scales rw[6],
        // d in rw[7].x.  Block g, half lh: codes from ql rw[2 (g & 1) + lh] (low nibble g < 2, high
        // g >= 2) and bits 2g of qh rw[4 + lh], minus 32; scale index 8 st + 2 g + lh
        if (st == 0) iacc = vNi<CM>{};
        const uint32_t scw[4] = { rw[6].x, rw[6].y, rw[6].z, rw[6].w };
        v4i an = a_op(0);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint4 half[2];
#pragma unroll
            for (int lh = 0; lh < 2; ++lh) {
                const uint4 ql = rw[2 * (g & 1) + lh], qh = rw[4 + lh];
                const int sh = g < 2 ? 0 : 4;
                auto code = [&](uint32_t l, uint32_t hb) {
                    const uint32_t c = ((l >> sh) & 0x0F0F0F0Fu) | (((hb >> (2 * g)) & 0x03030303u) << 4);
                    return ((c | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
                };
                half[lh] = make_uint4(code(ql.x, qh.x), code(ql.y, qh.y), code(ql.z, qh.z), code(ql.w, qh.w));
            }
            v4i op0, op1;
            swap_halves(half[0], half[1], op0, op1);
            // the row scales of halves lh = 0, 1 in the output lanes (rows 0-31: s?0, 32-63: s?1)
            const int is0 = 8 * st + 2 * g, is1 = is0 + 1;
            uint32_t a0, a1, b0, b1;
            swap_rows((scw[is0 >> 2] >> (8 * (is0 & 3))) & 0xffu, a0, a1);
            swap_rows((scw[is1 >> 2] >> (8 * (is1 & 3))) & 0xffu, b0, b1);
            const v4i av = an;
            if (g + 1 < 4) an = a_op(g + 1);
            const v4i z = v4i{};
            const v16i l0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, h ? z : op0, v16i{}, 0, 0, 0);
            const v16i l1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, h ? z : op1, v16i{}, 0, 0, 0);
            scale_add<NR>(l0, l1, (int)(int8_t)a0, (int)(int8_t)a1, iacc);
            __builtin_amdgcn_sched_barrier(0);
            const v16i u0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, h ? op0 : z, v16i{}, 0, 0, 0);
            const v16i u1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, h ? op1 : z, v16i{}, 0, 0, 0);
            scale_add<NR>(u0, u1, (int)(int8_t)b0, (int)(int8_t)b1, iacc);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (st == 1) {                                            // the super-block's float combine
            float dx0[NR];
            dx_op(0, dx0);
            uint32_t dd0, dd1;
            swap_rows(rw[7].x & 0xffffu, dd0, dd1);
            const float d[2] = { h2f(dd0), h2f(dd1) };
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < NR; ++r) out[NR * t + r] += dx0[r] * (d[t] * (float)iacc[NR * t + r]);
        }
    } else if constexpr (IQ) {
        const uint32_t shi = rw[8].x >> 16, slo = rw[8].y;
        const Iq4Regs kr = iq4_regs();                        // the codebook in VGPRs
        vNi<CM> isum = {};
        v16i pe0, pe1;
        int ps0 = 0, ps1 = 0;
        v4i an = a_op(0);                                     // LDS reads one block ahead
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            v4i op0, op1;
            uint4 lo, hi;
            iq4_map8(rw[ib], kr, lo, hi);
            swap_halves(lo, hi, op0, op1);
            uint32_t s0, s1;
            swap_rows(((slo >> (4 * ib)) & 0xFu) | (((shi >> (2 * ib)) & 3u) << 4), s0, s1);
            const v4i av = an;
            if (ib + 1 < 8) an = a_op(ib + 1);
            const v16i e0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, op0, v16i{}, 0, 0, 0);
            const v16i e1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, op1, v16i{}, 0, 0, 0);
            if (ib > 0) scale_add<NR>(pe0, pe1, ps0, ps1, isum);
            __builtin_amdgcn_sched_barrier(0);
            pe0 = e0;
            pe1 = e1;
            ps0 = (int)s0 - 32;
            ps1 = (int)s1 - 32;
        }
        scale_add<NR>(pe0, pe1, ps0, ps1, isum);
        float dx0[NR];
        dx_op(0, dx0);
        uint32_t dd0, dd1;
        swap_rows(rw[8].x & 0xffffu, dd0, dd1);
        const float d[2] = { h2f(dd0), h2f(dd1) };
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < NR; ++r) out[NR * t + r] += dx0[r] * (d[t] * (float)isum[NR * t + r]);
    }
}

// A work-group is TW tiles x WK waves: wave (tw, kw) = wave % TW, wave / TW streams tile
// tb TW + tw over the groups [gw + kw spw, + spw) of the work-group's K range [gw, gw + WK spw)
// (K slice ks of KS).  The K range's activations (CM columns) are staged once in LDS for all TW
// tiles, the WK waves of a tile are added in LDS in a fixed order, and KS > 1 adds into zeroed
// dst with atomics.  Weights stream through two register sets: stage s + 1 loads while s
// computes.
template <int TYPE, int CM>
__device__ __forceinline__ void gemv_mma_body(const GemvParams & p) {
    using T = GV<TYPE>;
    constexpr int NL = T::NL, NST = T::NST, NR = CM / 2;
    constexpr bool KQ = TYPE == QMM_TYPE_Q4_K, Q8 = TYPE == QMM_TYPE_Q8_0;
    constexpr bool BF = TYPE == QMM_TYPE_Q4_0 || Q8 || TYPE == QMM_TYPE_IQ4_NL;   // a float scale per 32 weights
    constexpr int BS = BF ? 32 : 256;                             // activation scale block
    constexpr int NSB = BF ? 8 : 1;                               // activation scales per group
    constexpr int kMagic = 0x4B400000;                            // float 12582912: its bits + i = 12582912 + i
    // LDS: 256 zero bytes (the A operand of lanes without a column), [WK spw][CM][kMmaColBytes]
    // codes, for Q4_K [WK spw][CM][16] split sums, then the activation scales [WK spw][NSB][CM];
    // after the stream, the waves' sums
    extern __shared__ __align__(16) uint8_t xl[];
    __shared__ int64_t s_col[CM], s_doff[CM];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int TW = p.tw, WK = p.W / p.tw;
    const int tw = wave % TW, kw = wave / TW;
    // work-group -> (task, tile block, K slice); these counts fit 32 bits
    static_assert(T::kReadEnd <= tile_group_bytes(TYPE) && tile_group_bytes(TYPE) <= (int)kSinkBytes,
                  "a stage reads inside one tile-group, which fits in the sink");
    const uint32_t ntl = (uint32_t)p.w.ntiles;
    // the grid (KS, tile blocks, tasks) is the position, as in k_gemv
    const uint32_t ks = blockIdx.x, tb = blockIdx.y, task = blockIdx.z + (uint32_t)p.task0;
    int mat, nc;
    bool sec = false;                  // the second image (gate/up in one launch)
    if (p.tasks) {
        uint32_t tk = task;
        if (p.base2 && p.glu < 0 && p.ntasks_dev && (int)tk >= *p.ntasks_dev) {  // the second pass over the list
            tk -= (uint32_t)*p.ntasks_dev;
            sec = true;
        }
        if (p.ntasks_dev && (int)tk >= *p.ntasks_dev) return;     // uniform
        const GemvTask & t = p.tasks[tk];
        const int64_t dadd = sec ? p.up_doff : 0;
        mat = t.mat;
        nc = t.ncols < kMaxTaskCols ? t.ncols : kMaxTaskCols;
        if (mat < 0) {                                            // pairs of invalid ids: zero rows
            const uint32_t ztile = tb * (uint32_t)TW + (uint32_t)tw;
            const int64_t row = (int64_t)ztile * kTileRows + lane;
            if (ks == 0 && kw == 0 && ztile < ntl && row < p.w.M)
                for (int j = 0; j < nc; ++j) p.dst[t.c[j].dst_off + dadd + row] = 0.0f;
            return;                                               // uniform
        }
        if (tid < nc) {
            s_col[tid] = t.c[tid].col;
            s_doff[tid] = t.c[tid].dst_off + dadd;
        }
    } else {
        const DenseTask dt = task == 0 ? DenseTask{ 0, 0, 0, 0, 0 }
                                       : dense_task(task, (uint32_t)p.tpb, (uint32_t)p.ne12, (uint32_t)p.r2,
                                                    (uint32_t)p.r3, (uint32_t)p.ne02);
        mat = dt.mat;
        if (p.base2 && mat == 1) {                                // gate/up in one launch
            mat = 0;
            sec = true;
        }
        const int64_t first = (int64_t)dt.tt * p.nct;
        nc = (int)((p.ne11 - first) < p.nct ? (p.ne11 - first) : p.nct);
        if (tid < nc) {
            const int64_t i1 = first + tid;
            s_col[tid] = (int64_t)dt.b * p.col_bs + i1;
            s_doff[tid] = i1 * p.d_nb1 + (int64_t)dt.i2 * p.d_nb2 + (int64_t)dt.i3 * p.d_nb3;
        }
    }
    if (mat < 0 || nc <= 0) return;                               // uniform
    const int G = (int)p.w.G;
    // the work-group's groups [gw, gw + ngw) (ngw >= 1: the plan leaves no empty slice), this
    // wave's [ga, ga + nsw)
    int gw, ngw, ga, nsw;
    mma_groups((int)ks, WK, kw, p.spw, G, gw, ngw, ga, nsw);
    const uint32_t tile = tb * (uint32_t)TW + (uint32_t)tw;
    const int S = tile < ntl ? nsw * NST : 0;                     // stages (uniform per wave)
    const uint8_t * tbase = mat_tile(p, mat, tile < ntl ? tile : 0, sec);   // the up tile after the gate (GLU)
    const size_t tgs = (size_t)p.w.tg;
    const bool glu = CM == 8 && p.glu >= 0;                       // uniform (lists: 8-column tasks only)
    // past the last stage: the sink, every lane at lane 0's address (one line per load
    // instruction instead of 16; the loads stay unconditional, so every wait counts both buffers)
    auto load_stage = [&](uint4 (&b)[NL], int s) {
        const bool real = s < S;
        T::load(b, real ? tbase + (size_t)stage_group(ga, s, NST) * tgs : p.sink, real ? s % NST : 0, real ? lane : 0);
    };
    // the first stage's weights are requested before the activations are staged
    uint4 b0[NL], b1[NL];
    if (S > 0) load_stage(b0, 0);
    __syncthreads();                                              // s_col, s_doff
    nc = __builtin_amdgcn_readfirstlane(nc);
    // the work-group's activation codes, Q4_K split sums and scales into LDS (zeros for columns >= nc)
    const int nthr = 64 * p.W;
    uint8_t * const xcl = xl + kMmaZeroBytes;
    if (tid < kMmaZeroBytes / 16) *reinterpret_cast<uint4 *>(xl + 16 * tid) = make_uint4(0, 0, 0, 0);
    for (int i = tid; i < ngw * CM * 16; i += nthr) {
        const int q = i & 15, c = (i >> 4) % CM, g = (i >> 4) / CM;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (c < nc) v = *reinterpret_cast<const uint4 *>(p.xc + s_col[c] * p.ldk + (int64_t)(gw + g) * 256 + 16 * q);
        *reinterpret_cast<uint4 *>(xcl + (g * CM + c) * kMmaColBytes + 16 * q) = v;
    }
    const int per = WK * p.spw;                                   // groups the LDS holds
    uint8_t * const xsl = xcl + per * CM * kMmaColBytes;
    if constexpr (KQ) {
        for (int i = tid; i < ngw * CM; i += nthr) {
            const int g = i / CM, c = i % CM;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (c < nc) v = *reinterpret_cast<const uint4 *>(p.bsp + ((int64_t)(gw + g) * p.ldT + s_col[c]) * 16);
            *reinterpret_cast<uint4 *>(xsl + 16 * i) = v;
        }
    }
    float * const xdl = reinterpret_cast<float *>(xsl + (KQ ? per * CM * 16 : 0));
    for (int i = tid; i < ngw * NSB * CM; i += nthr) {
        const int c = i % CM, gb = i / CM;                        // gb = group * NSB + block
        xdl[i] = c < nc ? p.xd[s_col[c] * (p.ldk / BS) + (int64_t)gw * NSB + gb] : 0.0f;
    }
    __syncthreads();
    const int h = lane >> 5, l32 = lane & 31;
    // A operand: the lane's column l32 (zeros past nc), k half h.  Lanes without a column read
    // the zero block (every offset stays inside its 256 bytes).
    const bool a_live = l32 < nc;
    const uint8_t * xar = a_live ? xcl + ((ga - gw) * CM + l32) * kMmaColBytes + 16 * h : xl;
    const int xas = a_live ? CM * kMmaColBytes : 0;               // per group
    // Q4_K min term: the split sums of the lane's column (lane half 0; zeros elsewhere)
    const bool s_live = KQ && a_live && h == 0;
    const uint8_t * xsr = s_live ? xsl + ((ga - gw) * CM + l32) * 16 : xl;
    const int xss = s_live ? CM * 16 : 0;
    // the scales of the lane's output columns (quads 8 q + 4 h), per (group, block)
    const float * xdr = xdl + (ga - gw) * NSB * CM + 4 * h;
    vNf<CM> out = {};
    vNi<CM> iacc = {};                                            // Q6_K: the super-block's integer sum
    v16i magic;
#pragma unroll
    for (int r = 0; r < 16; ++r) magic[r] = kMagic;
    auto compute = [&](const uint4 (&b)[NL], int s) {
        const int gl = s / NST;
        mma_stage<TYPE, CM, NL>(b, s % NST, xar + gl * xas, xdr + gl * NSB * CM, xsr + gl * xss, h, magic, out, iacc);
    };
    auto run = [&]() {
        for (int s = 0; s < S; s += 2) {                          // uniform
            load_stage(b1, s + 1);
            __builtin_amdgcn_sched_barrier(0);                    // the loads go out before the compute
            compute(b0, s);
            if (s + 1 >= S) break;
            load_stage(b0, s + 2);
            __builtin_amdgcn_sched_barrier(0);
            compute(b1, s + 1);
        }
    };
    run();
    vNf<CM> outu = {};
    if (glu) {                                                    // the up tile against the same activations
        const vNf<CM> outg = out;
        out = vNf<CM>{};
        tbase = mat_tile(p, mat, tile < ntl ? tile : 0, true);
        if (S > 0) load_stage(b0, 0);
        run();
        outu = out;
        out = outg;
    }

    // tile tw's WK waves are added in a fixed order (wave kw takes the elements e = kw, kw + WK,
    // ... of the CM), then stored (KS == 1) or added (KS > 1)
    const int64_t row0 = (int64_t)tile * kTileRows + l32;
    auto store = [&](int e, float v) {
        const int c = mma_col(e % NR, h);
        const int64_t row = row0 + 32 * (e / NR);
        if (tile < ntl && c < nc && row < p.w.M) {
            float * o = p.dst + s_doff[c] + row;
            if (p.KS == 1) *o = v;
            else atomicAdd(o, v);
        }
    };
    if (WK == 1) {
#pragma unroll
        for (int e = 0; e < CM; ++e) store(e, glu ? glu_apply(p.glu, out[e], outu[e]) : out[e]);
        return;
    }
    // [WK][TW][NV][64] over the staged data (NV = CM, with the GLU 2 CM: gate, then up)
    const int NV = glu ? 2 * CM : CM;
    float * red = reinterpret_cast<float *>(xl);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < CM; ++e) red[((kw * TW + tw) * NV + e) * 64 + lane] = out[e];
    if (glu) {
#pragma unroll
        for (int e = 0; e < CM; ++e) red[((kw * TW + tw) * NV + CM + e) * 64 + lane] = outu[e];
    }
    __syncthreads();
    for (int e = kw; e < CM; e += WK) {
        float v = 0.0f, u = 0.0f;
        for (int k = 0; k < WK; ++k) v += red[((k * TW + tw) * NV + e) * 64 + lane];
        if (glu) {
            for (int k = 0; k < WK; ++k) u += red[((k * TW + tw) * NV + CM + e) * 64 + lane];
            v = glu_apply(p.glu, v, u);
        }
        store(e, v);
    }
}

// 8 columns run three waves per SIMD; 16 and 32 (more accumulators: 16 spills 3 to 17
// registers at three waves) two
template <int TYPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_gemv_mma(GemvParams p) {
    gemv_mma_body<TYPE, 8>(p);
}
template <int TYPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_gemv_mma16(GemvParams p) {
    gemv_mma_body<TYPE, 16>(p);
}
template <int TYPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_gemv_mma32(GemvParams p) {
    gemv_mma_body<TYPE, 32>(p);
}

template <int TYPE>
hipError_t launch_t(const GemvParams & p0, int nc, int64_t nwg, hipStream_t s, const KTime * kt) {
    const int threads = 64 * p0.W;
    const size_t lds = p0.W > 1 ? (size_t)p0.W * nc * 64 * sizeof(float) * (p0.glu >= 0 ? 2 : 1) : 0;
    GemvParams p = p0;
    const int64_t per_task = (int64_t)p.KS * p.w.ntiles, ntasks = nwg / per_task;
    if (ntasks * per_task != nwg || p.w.ntiles > 65535) return hipErrorInvalidValue;
    // grid (KS, tiles, tasks): one launch per 65535 tasks (kernel timing stamps the first)
    for (int64_t t0 = 0; t0 < ntasks; t0 += 65535) {
        p.task0 = (int)t0;
        const dim3 g((unsigned)p.KS, (unsigned)p.w.ntiles, (unsigned)std::min<int64_t>(65535, ntasks - t0));
        const KTime * k = t0 == 0 ? kt : nullptr;
        switch (nc) {
#define QMM_NC(N)                                                                                  \
    case N:                                                                                        \
        if (k) hipExtLaunchKernelGGL(k_gemv<TYPE, N>, g, dim3(threads), (uint32_t)lds, s, k->start, k->stop, 0, p); \
        else k_gemv<TYPE, N><<<g, threads, lds, s>>>(p);                                           \
        break;
            QMM_NC(1) QMM_NC(2) QMM_NC(3) QMM_NC(4) QMM_NC(5) QMM_NC(6) QMM_NC(7) QMM_NC(8)
#undef QMM_NC
            default: return hipErrorInvalidValue;
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

int env_int(const char * name, int dflt) {
    const char * e = getenv(name);
    return e ? atoi(e) : dflt;
}

// ---- the v_dot4 GEMV with its own activation quantization (one launch per op) -------------
// k_gemv needs the pre-pass: a launch that quantizes src1 (and zeroes dst for its K slices'
// atomics) ahead of it.  At decode that launch and its kernel boundary are a fifth of the op.
// Here every wave quantizes the groups it streams itself, with the pre-pass's own quantizers
// (so the codes equal ggml-cpu's), into its own LDS slots, after its first weight stage is on
// its way; K is split among the waves of a work-group and added in LDS, so every output is
// stored once and nothing has to be zeroed first.  A dense product may also split K over KS
// work-groups per tile (one tile per work-group puts 272 work-groups of config 2's 17408-row
// matrices on 256 CUs, 16 of which then stream twice): the work-groups' sums meet in a
// pairwise tree of exchanges (tree_add) and the last arrival stores the row.  The same kernel
// takes:
//  * dense MUL_MAT at 1 or 2 columns per task, K split over KS >= 1 work-groups;
//  * MUL_MAT_ID at small batches with no route: task p is the (token, slot) pair p and reads its
//    expert id itself (the reference's per-pair matvec below 16 tokens, P01:1189-1192 and
//    P01:1222-1248); a negative id writes a zero row, an id past the stack too and sets the
//    error flag;
//  * either of them for a gate/up pair with its GLU: the work-group streams the gate tile, then
//    the up tile against the same quantized activations, and stores act(gate) * up;
//  * a MoE FFN block's two products (qmm_moe_ffn): pairs may add a shared-expert slot (slot
//    n_used of every token, its own images, no id), and the down product combines: each pair's
//    row is scaled by its router weight (the shared slot's by the sigmoid of its gate logit),
//    the token's slots meet in the exchange tree, and the root stores the token's output row;
//    the gate/up launch may rank the tokens' router logits itself (ROUTE: the work-group's first
//    wave runs topk_wave before the weight stream, whose addresses need the expert).
constexpr int kFqSlot = 320;   // one (group, column): 256 codes, 8 f32 scales at 256, 16 i16 sums at 288
constexpr int kFqMaxWaves = 16;

template <int N>
struct XL {
    static constexpr int NC = N;
    const int8_t * c[N];
    const float * d[N];
    const int16_t * s[N];
    __device__ static uint4 c4(const int8_t * p, int i) { return *reinterpret_cast<const uint4 *>(p + 4 * i); }
    __device__ static float df(const float * p, int i) { return p[i]; }
    __device__ static int s16(const int16_t * p, int i) { return p[i]; }
};

struct FqParams {
    WView w;
    F32Cols x;
    int64_t K;
    // dense tasks (ids == null): as k_gemv's
    int64_t ne11, ne12, r2, r3, ne02, tpb, col_bs;
    int64_t d_nb1, d_nb2, d_nb3;
    // MUL_MAT_ID pairs: pair p = t n_used + i, its id at t ids_nb1 + i ids_nb0 (bytes), its
    // activation column (i % ne11i) + t ne11i, its dst floats t dnb2 + i dnb1
    const char * ids;
    int64_t ids_nb0, ids_nb1, n_used, ne11i, n_as, dnb1, dnb2;
    int32_t * bad_id;
    float * dst;
    const uint8_t * sink;
    const uint8_t * base2;       // glu >= 0: the up image, w's shape
    int glu;
    int W, spw;
    int KS;                      // dense: work-groups per tile along K (grid z)
    uint32_t * tree;             // KS > 1: slots [task][tile][2 KS nodes][NC][64] (64-bit pairs with the GLU);
                                 // combine: [token][tile][2 slots nodes][64]
    // MoE FFN: a shared-expert slot after the n_used routed ones (its images: the gate / only
    // matrix and the up one, w's shape); combine: slot i of token t weighted by
    // cw[t cw_nb1 + i cw_nb0] (the shared slot by sigmoid(sl[t sl_nb1]), 1 without sl), the
    // token's row stored at dst + t d_nb1 (comb 1: the slots meet in the tree; comb 2: wave i
    // of the tile's work-group is slot i, the rows added in slot order through LDS)
    int n_shared;
    const uint8_t * sh_base;
    const uint8_t * sh_base2;
    int comb;
    const float * cw;
    int64_t cw_nb0, cw_nb1;
    const float * sl;
    int64_t sl_nb1;
    // MoE FFN with its router (the ROUTE kernel): the first wave of every work-group ranks its
    // token's logits (lg + t lg_nb1, n_expert of them) and takes its slot's expert from the
    // ranking; the work-groups of tile 0, slot 0 store the token's ids and weights (ids + t
    // ids_nb1 bytes, wout + t wout_nb1 floats) for the down launch
    const float * lg;
    int64_t lg_nb1;
    int n_expert;
    float cmin, cmax;
    float * wout;
    int64_t wout_nb1;
};

// The K slices of a tile add their sums v[j] (column j, this lane's row) up a pairwise tree
// in slot memory: at a level of n nodes, node i meets node i ^ 1 in slot (i / 2) of the
// level (an odd last node moves up alone).  Each meeting is one exchange: the first arrival
// leaves its sum in the slot and is done; the second takes it, adds it to its own (the
// sum of the two is the same whichever arrives first) and puts the slot back to kTreeEmpty.
// The last arrival at the root holds the row's total: alive[j] stays true for that lane
// only.  Every slot is reached by exactly two exchanges, so the protocol needs no ordering
// between different slots, and the launch ends with every slot empty again.
template <int NC>
__device__ __forceinline__ void tree_add(uint32_t * nodes, int ks, int KS, int nc, float (&v)[NC], bool (&alive)[NC],
                                         int lane) {
    uint32_t i = (uint32_t)ks, n = (uint32_t)KS, off = 0;
    while (n > 1) {                                               // uniform
        if ((i ^ 1u) < n) {
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                if (j < nc && alive[j]) {
                    uint32_t * s = nodes + ((size_t)(off + (i >> 1)) * NC + j) * 64 + lane;
                    const uint32_t o = __hip_atomic_exchange(s, __float_as_uint(v[j]), __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT);
                    if (o == kTreeEmpty) {
                        alive[j] = false;
                    } else {
                        v[j] += __uint_as_float(o);
                        __hip_atomic_store(s, kTreeEmpty, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
        }
        off += (n + 1) >> 1;
        i >>= 1;
        n = (n + 1) >> 1;
    }
}

// The same tree for a gate sum a[j] and an up sum b[j] (the GLU applied at the root): the pair
// travels as one 64-bit exchange (gate in the low word), so both meet the same partner at every
// node and the root holds both totals.  A gate sum is never the sentinel, so the low word says
// whether the slot was empty.
template <int NC>
__device__ __forceinline__ void tree_add_pairs(uint64_t * nodes, int ks, int KS, int nc, float (&a)[NC], float (&b)[NC],
                                               bool (&alive)[NC], int lane) {
    constexpr uint64_t kEmpty2 = ((uint64_t)kTreeEmpty << 32) | kTreeEmpty;
    uint32_t i = (uint32_t)ks, n = (uint32_t)KS, off = 0;
    while (n > 1) {                                               // uniform
        if ((i ^ 1u) < n) {
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                if (j < nc && alive[j]) {
                    uint64_t * s = nodes + ((size_t)(off + (i >> 1)) * NC + j) * 64 + lane;
                    const uint64_t mine = (uint64_t)__float_as_uint(a[j]) | ((uint64_t)__float_as_uint(b[j]) << 32);
                    const uint64_t o = __hip_atomic_exchange(s, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if ((uint32_t)o == kTreeEmpty) {
                        alive[j] = false;
                    } else {
                        a[j] += __uint_as_float((uint32_t)o);
                        b[j] += __uint_as_float((uint32_t)(o >> 32));
                        __hip_atomic_store(s, kEmpty2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
        }
        off += (n + 1) >> 1;
        i >>= 1;
        n = (n + 1) >> 1;
    }
}

// this lane's 4 activations of group g of column col (zeros past K; the loads stay inside the
// column and take no branch, so the waits that follow can count them)
__device__ __forceinline__ void load_x4(const F32Cols & xs, int64_t K, int64_t col, int g, int lane, float (&v)[4]) {
    const int64_t k = (int64_t)g * 256 + 4 * lane;                // K is whole 32-blocks (q8_0) or 256-blocks
    const bool in = k < K;
    const float * x = f32_col(xs, col) + (in ? k : 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float t = x[i];
        v[i] = in ? t : 0.f;
    }
}

// group g of activation column col, quantized by one wave into a slot (the pre-pass's quantizers)
// from the lanes' 4 values each (load_x4)
template <int VDT>
__device__ __forceinline__ void quant_slot(float (&v)[4], uint8_t * slot, int lane) {
    float d;
    int s;
    if constexpr (VDT == QMM_TYPE_Q8_K) {
        const uint32_t q = quant_q8_K_wave(v, lane, &d, &s);
        reinterpret_cast<uint32_t *>(slot)[lane] = q;
        if ((lane & 3) == 0) reinterpret_cast<int16_t *>(slot + 288)[lane >> 2] = (int16_t)s;
        if (lane == 0) reinterpret_cast<float *>(slot + 256)[0] = d;
    } else {
        const uint32_t q = quant_q8_0_lane(v, &d, &s);
        reinterpret_cast<uint32_t *>(slot)[lane] = q;
        if ((lane & 7) == 0) {
            reinterpret_cast<float *>(slot + 256)[lane >> 3] = d;
            reinterpret_cast<int16_t *>(slot + 288)[lane >> 3] = (int16_t)s;
        }
    }
}

// A work-group is W waves on one 64-row tile of one task, wave w streaming groups
// [w spw, w spw + spw) (dot4_stages with one K slice).  LDS: the waves' slots [W][spw][NC], then,
// after the stream, the waves' sums [W][NV][64].
template <int TYPE, int NC, bool ROUTE = false>
__global__ __launch_bounds__(1024) void k_gemv_fq(FqParams p) {
    using T = GV<TYPE>;
    constexpr int NL = T::NL, NST = T::NST;
    constexpr int VDT = (TYPE == QMM_TYPE_Q4_0 || TYPE == QMM_TYPE_Q8_0 || TYPE == QMM_TYPE_IQ4_NL) ? QMM_TYPE_Q8_0
                                                                                                     : QMM_TYPE_Q8_K;
    static_assert(T::kReadEnd <= tile_group_bytes(TYPE) && tile_group_bytes(TYPE) <= (int)kSinkBytes,
                  "a stage reads inside one tile-group, which fits in the sink");
    extern __shared__ __align__(16) uint8_t sm[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // the grid is the position: (tiles, slots, tokens) for MUL_MAT_ID pairs, pair p = t n_used + i;
    // (tiles, tasks, K slices) for dense products
    const uint32_t tile = blockIdx.x, task = blockIdx.y;
    const int ks = p.ids ? 0 : (int)blockIdx.z;
    int mat, nc;
    int64_t colv[NC], doffv[NC];
    bool shared = false, skip = false;
    const int G = (int)p.w.G;
    // combine mode 2 (MoE down, slots as waves): wave w is slot w of the token over the whole K
    const bool slotw = p.comb == 2;                               // uniform
    int ga, S;
    dot4_stages(ks, slotw ? 1 : p.W, slotw ? 0 : wave, p.spw, G, NST, ga, S);
    // the wave's activation groups, quantized into its slots [group][column]
    float xv[NC][4];
    uint8_t * const slots = sm + (size_t)wave * p.spw * NC * kFqSlot;
    bool xq = false;                                              // the slots are filled
    auto quantize = [&]() {
        for (int gi = 0; gi * NST < S; ++gi) {                    // uniform
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                if (j < nc) {
                    if (gi > 0) load_x4(p.x, p.K, colv[j], ga + gi, lane, xv[j]);
                    quant_slot<VDT>(xv[j], slots + (gi * NC + j) * kFqSlot, lane);
                }
            }
        }
        xq = true;
    };
    if (p.ids) {
        const int64_t t = blockIdx.z, i = slotw ? wave : blockIdx.y;
        shared = i >= p.n_used;                                   // uniform (over the wave): the shared expert's slot
        nc = 1;
#pragma unroll
        for (int j = 0; j < NC; ++j) colv[j] = (i % p.ne11i) + t * p.ne11i;
        int32_t e = 0;
        if constexpr (ROUTE) {
            __shared__ uint32_t r_key[1024];
            __shared__ int r_exp[1024];
            __shared__ float r_p[32];
            __shared__ int32_t r_id[32];
            __shared__ float r_w[32];
            // the activations do not depend on the route: every wave requests its first group
            // before the ranking, and the waves that do not rank quantize theirs meanwhile
#pragma unroll
            for (int j = 0; j < NC; ++j) load_x4(p.x, p.K, colv[j], ga, lane, xv[j]);
            if (wave == 0)
                topk_wave_any(p.lg + t * p.lg_nb1, p.n_expert, (int)p.n_used, p.cmin, p.cmax, lane, r_key, r_exp, r_p,
                              r_id, r_w);
            else
                quantize();
            __syncthreads();
            if (!shared) e = r_id[i];
            if (tile == 0 && i == 0 && wave == 0 && lane < p.n_used) {
                reinterpret_cast<int32_t *>(const_cast<char *>(p.ids) + t * p.ids_nb1)[lane] = r_id[lane];
                p.wout[t * p.wout_nb1 + lane] = r_w[lane];
            }
        } else if (!shared) {
            e = *reinterpret_cast<const int32_t *>(p.ids + t * p.ids_nb1 + i * p.ids_nb0);
        }
        const int64_t doff = t * p.dnb2 + i * p.dnb1;
        if (e < 0 || e >= p.n_as) {                                // uniform: a zero row
            if ((slotw || wave == 0) && e >= p.n_as && tile == 0 && lane == 0) *p.bad_id = 1;
            if (!p.comb) {
                if (wave == 0) {
                    const int64_t row = (int64_t)tile * kTileRows + lane;
                    if (row < p.w.M) p.dst[doff + row] = 0.0f;
                }
                return;
            }
            skip = true;                                          // (combine: the slot still meets the others)
        }
        mat = skip || shared ? 0 : QMM_RED == 8 ? (int)((e + 1) % p.n_as) : e;   // (mutation 8: the next expert)
#pragma unroll
        for (int j = 0; j < NC; ++j) doffv[j] = doff;
    } else {
        const DenseTask dt = task == 0 ? DenseTask{ 0, 0, 0, 0, 0 }
                                       : dense_task(task, (uint32_t)p.tpb, (uint32_t)p.ne12, (uint32_t)p.r2,
                                                    (uint32_t)p.r3, (uint32_t)p.ne02);
        mat = dt.mat;
        const int64_t first = (int64_t)dt.tt * NC;
        nc = (int)((p.ne11 - first) < NC ? (p.ne11 - first) : NC);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int64_t i1 = first + (j < nc ? j : 0);
            colv[j] = (int64_t)dt.b * p.col_bs + i1;
            doffv[j] = i1 * p.d_nb1 + (int64_t)dt.i2 * p.d_nb2 + (int64_t)dt.i3 * p.d_nb3;
        }
    }
    nc = __builtin_amdgcn_readfirstlane(nc);
    if (skip) S = 0;                                              // (a zero row: no stages, no groups)
    const bool glu = p.glu >= 0;                                  // uniform
    const int ST = glu ? 2 * S : S;                               // gate stages, then up stages
    WView w1 = p.w, w2 = p.w;
    if (shared) w1.base = p.sh_base;
    w2.base = shared ? p.sh_base2 : p.base2;
    const uint8_t * tbg = tile_group(w1, mat, tile, 0);
    const uint8_t * tbu = glu ? tile_group(w2, mat, tile, 0) : tbg;
    const size_t tgs = (size_t)p.w.tg;
    // Two-stage types (Q6_K, Q8_0): both stages of a group are requested together (B, then B1),
    // so a wave of one group waits for one weight round trip, not two.
    uint4 B[NL], B1[NL];
    auto load_into = [&](uint4 (&dst)[NL], int s) {               // past the last stage: the sink
        const uint8_t * tg = p.sink;
        int st = 0;
        if (s < ST) {
            const int sl = s < S ? s : s - S;
            tg = (s < S ? tbg : tbu) + (size_t)stage_group(ga, sl, NST) * tgs;
            st = sl % NST;
        }
        T::load(dst, tg, st, lane);
    };
    auto load_stage = [&](int s) {
        load_into(B, s);
        if constexpr (NST == 2) load_into(B1, s + 1);
    };
    // the first group's activations are requested ahead of the weights: behind the weight
    // stream in the memory queues they would arrive with its end and hold every dot back
    // (both unconditional: colv[j] is a column of src1 for every j, a wave without groups reads
    // zeros and the sink; with a route they were requested before the ranking)
    if (!ROUTE) {
#pragma unroll
        for (int j = 0; j < NC; ++j) load_x4(p.x, p.K, colv[j], ga, lane, xv[j]);
    }
    load_stage(0);
    if (!xq) quantize();
    __builtin_amdgcn_wave_barrier();
    float acc[NC], accu[NC];
    int st_state[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        acc[j] = 0.0f;
        accu[j] = 0.0f;
        st_state[j] = 0;
    }
    for (int s = 0; s < ST; ++s) {                                // uniform
        const int sl = s < S ? s : s - S, gi = sl / NST;
        XL<NC> x;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const uint8_t * sj = slots + (gi * NC + j) * kFqSlot;
            x.c[j] = reinterpret_cast<const int8_t *>(sj);
            x.d[j] = reinterpret_cast<const float *>(sj + 256);
            x.s[j] = reinterpret_cast<const int16_t *>(sj + 288);
        }
        if constexpr (NST == 2) {                                 // (ST is even: whole groups)
            if (s < S) {
                T::dot(B, 0, x, nc, acc, st_state);
                T::dot(B1, 1, x, nc, acc, st_state);
            } else {
                T::dot(B, 0, x, nc, accu, st_state);
                T::dot(B1, 1, x, nc, accu, st_state);
            }
            ++s;
            if (s + 1 < ST) load_stage(s + 1);                    // (nothing past the last stage)
        } else {
            if (s < S) T::dot(B, sl % NST, x, nc, acc, st_state);
            else T::dot(B, sl % NST, x, nc, accu, st_state);
            if (s + 1 < ST) load_stage(s + 1);                    // (nothing past the last stage)
        }
    }
    const int64_t row = (int64_t)tile * kTileRows + lane;
    if (slotw) {                                                  // uniform (MoE down, one column)
        // each slot's row times its weight (rounded, as the graph's MUL), then the token's rows
        // added slot by slot, the routed ones in order and the gated shared expert last: the
        // graph's chain of ADDs
        const int64_t t = blockIdx.z;
        const int nsl = (int)(p.n_used + p.n_shared);
        float wgt;
        if (!shared) wgt = p.cw[t * p.cw_nb1 + (int64_t)wave * p.cw_nb0];
        else wgt = p.sl ? 1.0f / (1.0f + expf(-p.sl[t * p.sl_nb1])) : 1.0f;
        float * red = reinterpret_cast<float *>(sm);
        __syncthreads();                                          // every wave is done with its slots
        red[wave * 64 + lane] = __fmul_rn(acc[0], wgt);
        __syncthreads();
        if (wave != 0 || row >= p.w.M) return;
        float v = red[lane];
        for (int ww = 1; ww < nsl; ++ww) v = __fadd_rn(v, red[ww * 64 + lane]);
        p.dst[t * p.d_nb1 + row] = v;
        return;
    }
    // the W waves added in a fixed order: the gate (or only) sums tot[], with the GLU the up sums
    // totu[]; act(gate) * up once the K slices have met
    float tot[NC], totu[NC];
    if (p.W > 1) {
        const int NV = glu ? 2 * NC : NC;
        float * red = reinterpret_cast<float *>(sm);
        __syncthreads();                                          // every wave is done with the slots
#pragma unroll
        for (int j = 0; j < NC; ++j) red[(wave * NV + j) * 64 + lane] = acc[j];
        if (glu) {
#pragma unroll
            for (int j = 0; j < NC; ++j) red[(wave * NV + NC + j) * 64 + lane] = accu[j];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            float v = red[j * 64 + lane], u = 0.0f;
            for (int ww = 1; ww < p.W; ++ww) v += red[(ww * NV + j) * 64 + lane];
            if (glu) {
                u = red[(NC + j) * 64 + lane];
                for (int ww = 1; ww < p.W; ++ww) u += red[(ww * NV + NC + j) * 64 + lane];
            }
            tot[j] = v;
            totu[j] = u;
        }
    } else {
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            tot[j] = acc[j];
            totu[j] = accu[j];
        }
    }
    bool alive[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) alive[j] = true;
    if (p.KS > 1) {                                               // uniform (dense)
        uint32_t * nodes = p.tree + ((size_t)task * (size_t)p.w.ntiles + tile) * (2 * (size_t)p.KS * NC * 64) * (glu ? 2 : 1);
        if (glu) tree_add_pairs<NC>(reinterpret_cast<uint64_t *>(nodes), ks, p.KS, nc, tot, totu, alive, lane);
        else tree_add<NC>(nodes, ks, p.KS, nc, tot, alive, lane);
    }
    if (p.comb) {                                                 // uniform (MoE down, one column)
        // the slot's row times its weight (each product rounded, as the graph's MUL), then the
        // token's slots added in the tree; every slot of every tile takes part, so each node
        // sees its two exchanges and the launch leaves the slots empty
        const int64_t t = blockIdx.z, i = blockIdx.y, nsl = p.n_used + p.n_shared;
        float wgt;
        if (!shared) wgt = p.cw[t * p.cw_nb1 + i * p.cw_nb0];
        else wgt = p.sl ? 1.0f / (1.0f + expf(-p.sl[t * p.sl_nb1])) : 1.0f;
#pragma unroll
        for (int j = 0; j < NC; ++j) tot[j] = __fmul_rn(tot[j], wgt);
        uint32_t * nodes = p.tree + ((size_t)t * (size_t)p.w.ntiles + tile) * (2 * (size_t)nsl * 64);
        tree_add<NC>(nodes, (int)i, (int)nsl, 1, tot, alive, lane);
        if (row >= p.w.M || !alive[0]) return;
        p.dst[t * p.d_nb1 + row] = tot[0];
        return;
    }
    if (row >= p.w.M) return;
#pragma unroll
    for (int j = 0; j < NC; ++j)
        if (j < nc && alive[j]) p.dst[doffv[j] + row] = glu ? glu_apply(p.glu, tot[j], totu[j]) : tot[j];
}

}  // namespace

bool gemv_fused_plan(int type, const WView & w, int nc, int64_t ntasks, int target, FusedPlan * pl) {
    // (the launch's grid takes the tasks, or a MUL_MAT_ID's slots and tokens, as a dimension)
    if (!type_layout(type) || nc < 1 || nc > 2 || ntasks <= 0 || ntasks > 65535 || w.G <= 0 || w.ntiles <= 0)
        return false;
    const int64_t tiles = ntasks * w.ntiles;
    int64_t W = std::min<int64_t>(std::min<int64_t>(kFqMaxWaves, w.G), std::max<int64_t>(1, (target + tiles - 1) / tiles));
    const int64_t spw = (w.G + W - 1) / W;
    W = (w.G + spw - 1) / spw;                                    // no wave without groups
    pl->nc = nc;
    pl->ntasks = ntasks;
    pl->W = (int)W;
    pl->spw = (int)spw;
    pl->KS = 1;
    pl->lds = std::max<int64_t>(W * spw * nc * kFqSlot, W * 2 * nc * 64 * 4);
    return pl->lds <= 64 * 1024 && tiles < 0x7fffffff;
}

bool gemv_fused_split_plan(int type, const WView & w, int nc, int64_t ntasks, int W, int spw, FusedPlan * pl) {
    if (!type_layout(type) || nc < 1 || nc > 2 || ntasks <= 0 || ntasks > 65535 || w.G <= 0 || w.ntiles <= 0 ||
        W < 1 || W > kFqMaxWaves || spw < 1)
        return false;
    const int64_t per_wg = (int64_t)W * spw;
    const int64_t KS = (w.G + per_wg - 1) / per_wg;               // the last slice may have idle waves
    if (KS < 2 || KS > 65535) return false;
    pl->nc = nc;
    pl->ntasks = ntasks;
    pl->W = W;
    pl->spw = spw;
    pl->KS = (int)KS;
    pl->lds = std::max<int64_t>(per_wg * nc * kFqSlot, (int64_t)W * 2 * nc * 64 * 4);
    return pl->lds <= 64 * 1024 && ntasks * w.ntiles < 0x7fffffff;
}

bool gemv_fused_slot_plan(int type, const WView & w, int64_t nslots, int64_t T, FusedPlan * pl) {
    if (!type_layout(type) || nslots < 1 || nslots > kFqMaxWaves || T < 1 || T > 65535 || w.G <= 0 || w.ntiles <= 0)
        return false;
    pl->nc = 1;
    pl->ntasks = nslots * T;
    pl->W = (int)nslots;
    pl->spw = (int)w.G;
    pl->KS = 1;
    pl->lds = std::max<int64_t>(nslots * w.G * kFqSlot, nslots * 64 * 4);
    return pl->lds <= 64 * 1024 && T * w.ntiles < 0x7fffffff;
}

int64_t gemv_fused_tree_words(const WView & w, const FusedPlan & pl, bool glu) {
    return pl.KS > 1 ? pl.ntasks * w.ntiles * 2 * pl.KS * pl.nc * 64 * (glu ? 2 : 1) : 0;
}

int gemv_fused_waves_target() { return std::max(1, env_int("QMM_GEMV_FQ_WAVES", 4096)); }

hipError_t launch_gemv_fused(int type, const WView & w, const FusedPlan & pl, const FusedGemv & f, float * dst,
                             const void * sink, hipStream_t s, const KTime * kt) {
    if (!sink || !dst || pl.W < 1 || pl.W > kFqMaxWaves || pl.spw < 1 || pl.nc < 1 || pl.nc > 2 || pl.KS < 1 ||
        pl.KS > 65535 || (int64_t)pl.KS * pl.W * pl.spw < w.G ||
        (f.comb == 2 ? pl.KS != 1 || pl.spw < w.G || pl.W != f.n_used + f.n_shared
                     : pl.KS == 1 ? (int64_t)(pl.W - 1) * pl.spw >= w.G : (int64_t)(pl.KS - 1) * pl.W * pl.spw >= w.G) ||
        (pl.KS > 1 && (f.ids || !f.tree || ((uintptr_t)f.tree & 7))) || f.K != w.K ||
        (f.ids && (pl.nc != 1 || f.n_used < 1 || f.n_shared < 0 || f.n_shared > 1 ||
                   pl.ntasks != (f.n_used + f.n_shared) * f.T || !f.bad_id)) ||
        (!f.ids && (f.n_shared || f.comb)) || (f.n_shared && (!f.sh_base || (f.glu >= 0 && !f.sh_base2))) ||
        (f.comb && (pl.KS != 1 || (f.comb == 1 && !f.tree) || f.comb > 2 || !f.cw || f.glu >= 0 ||
                    (f.n_used + f.n_shared) * f.T * w.ntiles > 0x7fffffff)) ||
        (f.lg && (!f.ids || f.comb || !f.wout || f.n_expert < 1 || f.n_expert > 1024 || f.n_used > 32 ||
                  f.n_used > f.n_expert || f.ids_nb0 != 4 || f.n_as != f.n_expert)) ||
        (f.glu > QMM_GLU_GEGLU_QUICK) || (f.glu >= 0 && !f.base2))
        return hipErrorInvalidValue;
    FqParams p{};
    p.w = w;
    p.x = f.x;
    p.K = f.K;
    p.dst = dst;
    p.sink = (const uint8_t *)sink;
    p.base2 = f.base2;
    p.glu = f.glu;
    p.W = pl.W;
    p.spw = pl.spw;
    p.KS = pl.KS;
    p.tree = f.tree;
    if (f.ids) {
        p.ids = f.ids;
        p.ids_nb0 = f.ids_nb0;
        p.ids_nb1 = f.ids_nb1;
        p.n_used = f.n_used;
        p.ne11i = f.ne11;
        p.n_as = f.n_as;
        p.dnb1 = f.dnb1;
        p.dnb2 = f.dnb2;
        p.bad_id = f.bad_id;
        p.n_shared = f.n_shared;
        p.sh_base = f.sh_base;
        p.sh_base2 = f.sh_base2;
        p.comb = f.comb;
        p.cw = f.cw;
        p.cw_nb0 = f.cw_nb0;
        p.cw_nb1 = f.cw_nb1;
        p.sl = f.sl;
        p.sl_nb1 = f.sl_nb1;
        p.d_nb1 = f.d_nb1;
        p.lg = f.lg;
        p.lg_nb1 = f.lg_nb1;
        p.n_expert = f.n_expert;
        p.cmin = f.cmin;
        p.cmax = f.cmax;
        p.wout = f.wout;
        p.wout_nb1 = f.wout_nb1;
    } else {
        const GemvDense & d = f.dense;
        p.ne11 = d.ne11;
        p.ne12 = d.ne12;
        p.r2 = d.r2;
        p.r3 = d.r3;
        p.ne02 = d.ne02;
        p.col_bs = d.col_bs < 0 ? d.ne11 : d.col_bs;
        p.tpb = (d.ne11 + pl.nc - 1) / pl.nc;
        p.d_nb1 = d.d_nb1;
        p.d_nb2 = d.d_nb2;
        p.d_nb3 = d.d_nb3;
        if (p.tpb * d.ne12 * d.ne13 != pl.ntasks) return hipErrorInvalidValue;
    }
    const int64_t nwg = pl.ntasks * w.ntiles;
    if (nwg <= 0 || nwg >= 0x7fffffff) return hipErrorInvalidValue;
    const dim3 g = f.ids ? dim3((unsigned)w.ntiles, f.comb == 2 ? 1u : (unsigned)(f.n_used + f.n_shared), (unsigned)f.T)
                         : dim3((unsigned)w.ntiles, (unsigned)pl.ntasks, (unsigned)pl.KS);
    if (w.ntiles > 0x7fffffff || (f.ids ? f.n_used + f.n_shared > 65535 || f.T > 65535 : pl.ntasks > 65535))
        return hipErrorInvalidValue;
    const dim3 b(64 * pl.W);
    const uint32_t lds = (uint32_t)pl.lds;
#define QMM_FQ_K(...)                                                                              \
    if (kt) hipExtLaunchKernelGGL(__VA_ARGS__, g, b, lds, s, kt->start, kt->stop, 0, p);            \
    else __VA_ARGS__<<<g, b, lds, s>>>(p);                                                          \
    return hipGetLastError();
#define QMM_FQ(T)                                                                                   \
    if (f.lg) { QMM_FQ_K(k_gemv_fq<T, 1, true>) }                                                   \
    if (pl.nc == 1) { QMM_FQ_K(k_gemv_fq<T, 1>) }                                                   \
    QMM_FQ_K(k_gemv_fq<T, 2>)
    switch (type) {
        case QMM_TYPE_Q4_0: { QMM_FQ(QMM_TYPE_Q4_0) }
        case QMM_TYPE_Q8_0: { QMM_FQ(QMM_TYPE_Q8_0) }
        case QMM_TYPE_Q4_K: { QMM_FQ(QMM_TYPE_Q4_K) }
        case QMM_TYPE_Q5_K: { QMM_FQ(QMM_TYPE_Q5_K) }
        case QMM_TYPE_Q6_K: { QMM_FQ(QMM_TYPE_Q6_K) }
        case QMM_TYPE_IQ4_XS: { QMM_FQ(QMM_TYPE_IQ4_XS) }
        case QMM_TYPE_IQ4_NL: { QMM_FQ(QMM_TYPE_IQ4_NL) }
        default: return hipErrorInvalidValue;
    }
#undef QMM_FQ
#undef QMM_FQ_K
}


bool gemv_mma_supported(int type) {
    return type == QMM_TYPE_Q4_0 || type == QMM_TYPE_Q8_0 || type == QMM_TYPE_Q4_K || type == QMM_TYPE_IQ4_XS ||
           type == QMM_TYPE_IQ4_NL || type == QMM_TYPE_Q6_K;
}

bool gemv_plan(int type, const WView & w, int nc, int64_t ntasks, bool allow_split, bool want_mma, GemvPlan * pl) {
    if (!type_layout(type) || nc < 1 || nc > kMmaMaxCols || ntasks <= 0 || w.G <= 0 || w.ntiles <= 0) return false;
    pl->nc = nc;
    pl->ntasks = ntasks;
    const int64_t tiles = ntasks * w.ntiles;
    // MFMA kernel: about `target` waves, one per tile and K slice, W tiles per work-group; a
    // slice stages at most kMmaMaxGroups groups of activations in LDS (task lists, which
    // cannot split K, fall back to the v_dot4 kernel past that)
    pl->mma = want_mma && gemv_mma_supported(type);
    pl->tw = 1;
    pl->cm = 8;
    if (nc < 1 || nc > (pl->mma ? kMmaMaxCols : kMaxTaskCols)) return false;
    if (pl->mma) {
        pl->cm = nc <= 8 ? 8 : nc <= 16 ? 16 : 32;
        const int64_t maxg = (int64_t)kMmaMaxGroups * 8 / pl->cm;   // the LDS stages cm columns per group
        // MFMA kernel: about `target` waves in work-groups of TW tiles x WK waves; the WK waves
        // of a tile split K and are added in LDS, which stages the work-group's activations
        // (WK spw <= kMmaMaxGroups groups); the rest of the split is KS work-groups per tile
        // (atomics).  Task lists cannot split K over work-groups and fall back to the v_dot4
        // kernel past WK spw = G.
        // by (tile, group) pairs (sweeps on the config shapes: 3584 pairs ran best at 1024
        // waves, 5440 at 2048, the 151936-row head's 47480 at 4096, 10 % under its time at
        // 2048); targets between these split the groups unevenly (3584 pairs at 1433 waves:
        // slices of 3, 3, 3, 3, 3, 1 groups, slower than either neighbour)
        const int64_t pairs = tiles * w.G;
        const int64_t tgw = pairs < 4096 ? 1024 : pairs < 16384 ? 2048 : 4096;
        const int64_t target = std::max(1, env_int("QMM_GEMV_MMA_WAVES", (int)tgw));
        // (at most 4 waves per work-group: three 4-wave work-groups fill a CU at the kernel's
        // occupancy of 3 waves per SIMD, 8-wave ones leave a third of it idle)
        const int64_t TW = std::min<int64_t>(std::max(1, std::min(4, env_int("QMM_GEMV_MMA_TILES", 4))), w.ntiles);
        const int64_t wkmax = std::max<int64_t>(1, std::min<int64_t>(env_int("QMM_GEMV_MMA_WK", 1), 4 / TW));
        const int64_t kw = std::min<int64_t>(w.G, std::max<int64_t>(1, (target + tiles - 1) / tiles));
        int64_t spw = (w.G + kw - 1) / kw;
        int64_t WK = std::min<int64_t>((w.G + spw - 1) / spw, allow_split ? wkmax : 4 / TW);
        spw = std::min<int64_t>(allow_split ? spw : (w.G + WK - 1) / WK, std::max<int64_t>(1, maxg / WK));
        int64_t KS = (w.G + spw * WK - 1) / (spw * WK);
        WK = std::min<int64_t>(WK, ((w.G + KS - 1) / KS + spw - 1) / spw);   // balance the slices
        KS = (w.G + spw * WK - 1) / (spw * WK);
        if (KS == 1 || allow_split) {
            pl->tw = (int)TW;
            pl->W = (int)(TW * WK);
            pl->KS = (int)KS;
            pl->spw = (int)spw;
            const int64_t nwg = gemv_workgroups(w, *pl);
            return nwg > 0 && nwg < 0x7fffffff;
        }
        pl->mma = false;
        pl->cm = 8;
        if (nc > kMaxTaskCols) return false;
    }
    // waves: about `target` in all (each with at least one group), at most
    // wmax per work-group; the rest of the split goes to work-groups per tile
    // (KS), which need dst zeroed before the launch
    // (8192: on config 2's 17408 x 5120 Q4_K that is 20 K slices of one group each, 2.5 % faster
    // per op than 10 slices of two since the position stopped costing divisions; within 1 % of
    // 4096 on every other decode shape of the configs)
    const int64_t target = std::max(1, env_int("QMM_GEMV_WAVES", 8192));
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
    const int64_t nwg = gemv_workgroups(w, *pl);
    return nwg > 0 && nwg < 0x7fffffff;
}

int64_t gemv_workgroups(const WView & w, const GemvPlan & pl) {
    const int64_t tw = pl.mma ? pl.tw : 1;
    return pl.ntasks * ((w.ntiles + tw - 1) / tw) * pl.KS;
}

size_t gemv_lds_bytes(int type, const GemvPlan & pl) {
    if (pl.mma) {
        const size_t cm = (size_t)pl.cm;
        const size_t per_group = cm * (kMmaColBytes + (type == QMM_TYPE_Q4_K ? 16 : 0)) +
                                 cm * sizeof(float) * (vec_dot_type(type) == QMM_TYPE_Q8_0 ? 8 : 1);
        const size_t stage = kMmaZeroBytes + (size_t)(pl.W / pl.tw) * pl.spw * per_group;
        const size_t red = pl.W > pl.tw ? (size_t)pl.W * cm * 64 * sizeof(float) : 0;   // the K waves' sums
        return std::max(stage, red);
    }
    return pl.W > 1 ? (size_t)pl.W * pl.nc * 64 * sizeof(float) : 0;
}

namespace {
template <int TYPE> constexpr int read_end_of() { return GV<TYPE>::kReadEnd; }
template <int TYPE> constexpr int nst_of() { return GV<TYPE>::NST; }
// (read extent of a stage from its tile-group base, stages per group) of a type; false if unknown
bool stage_shape(int type, int * read_end, int * nst) {
    switch (type) {
#define QMM_SS(T) case T: *read_end = read_end_of<T>(); *nst = nst_of<T>(); return true;
        QMM_SS(QMM_TYPE_Q4_0) QMM_SS(QMM_TYPE_Q8_0) QMM_SS(QMM_TYPE_Q4_K) QMM_SS(QMM_TYPE_Q5_K)
        QMM_SS(QMM_TYPE_Q6_K) QMM_SS(QMM_TYPE_IQ4_XS) QMM_SS(QMM_TYPE_IQ4_NL)
#undef QMM_SS
        default: return false;
    }
}
}  // namespace

// The loads a GEMV launch makes, replayed on the host with the kernels' own index functions
// (wg_pos, dense_task, dot4_stages / mma_groups, stage_group): every work-group and wave, its
// stages 0 .. S - 1 from the image and, for the MFMA kernel, the one stage S that its
// two-buffer ring loads past its end from the sink (loaded and never consumed).  The v_dot4
// kernels load no stage past their last; a wave of the fused kernel without groups (the last
// K slice of a split plan) loads one stage of the sink, which is not counted here.
bool gemv_extent(int type, const WView & w, const GemvPlan & pl, const GemvDense * dense, int64_t nmat, int list_mat,
                 GemvExtent * e) {
    int rend, nst;
    if (!e || !stage_shape(type, &rend, &nst) || w.tg != tile_group_bytes(type)) return false;
    *e = GemvExtent{};
    e->image_bytes = (int64_t)nmat * w.ntiles * w.G * w.tg;
    e->real_lo = INT64_MAX;
    e->read_end = rend;
    const int64_t nwg = gemv_workgroups(w, pl);
    const int G = (int)w.G;
    const uint32_t ntl = (uint32_t)w.ntiles, TW = pl.mma ? (uint32_t)pl.tw : 1u, ntb = (ntl + TW - 1) / TW;
    const int64_t tpb = dense ? (dense->ne11 + pl.nc - 1) / pl.nc : 0;
    auto wave_loads = [&](int mat, uint32_t tile, int ga, int S) {
        if (S <= 0) return;
        for (int s = 0; s < S; ++s) {
            const int g = stage_group(ga, s, nst);
            const int64_t off = ((mat * (int64_t)w.ntiles + tile) * w.G + g) * w.tg;
            if (mat < 0 || mat >= nmat || tile >= ntl || g < 0 || g >= G || off < 0 || off + rend > e->image_bytes) e->bad++;
            e->real_lo = std::min(e->real_lo, off);
            e->real_hi = std::max(e->real_hi, off + rend);
            e->real_loads++;
        }
        if (pl.mma) {                                             // stage S: the sink, at its base
            e->sink_hi = std::max<int64_t>(e->sink_hi, rend);
            e->sink_loads++;
        }
        if (rend > (int64_t)kSinkBytes) e->bad++;
    };
    for (int64_t b = 0; b < nwg; ++b) {
        const WgPos wp = wg_pos((uint32_t)b, (uint32_t)pl.KS, pl.mma ? ntb : ntl);
        int mat = list_mat;
        if (dense) {
            mat = dense_task(wp.task, (uint32_t)tpb, (uint32_t)dense->ne12, (uint32_t)dense->r2, (uint32_t)dense->r3,
                             (uint32_t)dense->ne02).mat;
            if (dense->base2 && mat == 1) mat = 0;                // the second image has the first's shape
        }
        if (pl.mma) {
            const int WK = pl.W / pl.tw;
            for (int wave = 0; wave < pl.W; ++wave) {
                int gw, ngw, ga, nsw;
                mma_groups((int)wp.ks, WK, wave / pl.tw, pl.spw, G, gw, ngw, ga, nsw);
                if (ngw < 1 || gw + ngw > G || ngw > WK * pl.spw) e->bad++;   // activation groups staged in LDS
                const uint32_t tile = wp.unit * TW + (uint32_t)(wave % pl.tw);
                wave_loads(mat, tile, ga, tile < ntl ? nsw * nst : 0);
            }
        } else {
            for (int wave = 0; wave < pl.W; ++wave) {
                int ga, S;
                dot4_stages((int)wp.ks, pl.W, wave, pl.spw, G, nst, ga, S);
                wave_loads(mat, wp.unit, ga, S);
            }
        }
    }
    if (!e->real_loads) e->real_lo = 0;
    return true;
}

hipError_t launch_gemv(int type, const WView & w, const GemvPlan & pl, const ActBuf & a, const GemvTask * tasks,
                       const int32_t * ntasks_dev, const GemvDense * dense, float * dst, const void * sink,
                       hipStream_t s, const KTime * kt, const GemvPair * pair) {
    if (!sink || (!tasks && !dense) || pl.W < 1 || pl.W > 8 || pl.KS < 1 || pl.spw < 1 || a.ldk != w.G * 256 ||
        a.vdt != vec_dot_type(type))
        return hipErrorInvalidValue;
    GemvParams p{};
    p.w = w;
    p.xc = a.codes;
    p.xd = a.d;
    p.xs = a.sums;
    p.bsp = a.bsp;
    p.ldT = a.ldT;
    p.ldk = a.ldk;
    p.tasks = tasks;
    p.ntasks_dev = ntasks_dev;
    p.dst = dst;
    p.sink = (const uint8_t *)sink;
    p.W = pl.W;
    p.KS = pl.KS;
    p.spw = pl.spw;
    p.nct = pl.nc;
    p.tw = pl.tw;
    p.glu = -1;
    p.sh_mat = -1;
    if (pair) {
        if (!tasks || !ntasks_dev || pair->glu > QMM_GLU_GEGLU_QUICK || (pair->glu >= 0 && !pair->base2) ||
            (pair->sh_mat >= 0 && (!pair->sh_base || (pair->base2 && !pair->sh_base2))))
            return hipErrorInvalidValue;
        p.base2 = pair->base2;
        p.up_doff = pair->up_doff;
        p.glu = pair->glu;
        p.sh_mat = pair->sh_mat;
        p.sh_base = pair->sh_base;
        p.sh_base2 = pair->sh_base2;
    }
    if (!tasks) {
        p.ne11 = dense->ne11;
        p.col_bs = dense->col_bs < 0 ? dense->ne11 : dense->col_bs;
        p.base2 = dense->base2;
        if (p.base2 && (dense->ne12 * dense->ne13 != 2 || dense->ne02 != 2 || dense->r2 != 1)) return hipErrorInvalidValue;
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
    const int64_t nwg = gemv_workgroups(w, pl);
    if (pl.mma) {
        const int64_t per_wg = (int64_t)(pl.W / pl.tw) * pl.spw;
        if (!gemv_mma_supported(type) || nwg >= 0x7fffffff || pl.W > 4 || pl.tw < 1 || pl.W % pl.tw ||
            (pl.cm != 8 && pl.cm != 16 && pl.cm != 32) || pl.nc > pl.cm || (tasks && pl.cm != 8) ||
            per_wg > kMmaMaxGroups * 8 / pl.cm ||
            per_wg * pl.KS < w.G || per_wg * (pl.KS - 1) >= w.G || (type == QMM_TYPE_Q4_K && !a.bsp))
            return hipErrorInvalidValue;
        uint32_t lds = (uint32_t)gemv_lds_bytes(type, pl);
        if (p.glu >= 0 && pl.W > pl.tw)                          // the K waves' sums of gate and up
            lds = std::max<uint32_t>(lds, (uint32_t)pl.W * (uint32_t)pl.cm * 64 * 4 * 2);
        // grid (KS, tile blocks, tasks): one launch per 65535 tasks (kernel timing stamps the first)
        const int64_t ntb = (w.ntiles + pl.tw - 1) / pl.tw, per_task = (int64_t)pl.KS * ntb, ntasks = nwg / per_task;
        if (ntasks * per_task != nwg || ntb > 65535) return hipErrorInvalidValue;
        const dim3 b(64 * pl.W);
#define QMM_MMA_K(K)                                                                                \
    for (int64_t t0 = 0; t0 < ntasks; t0 += 65535) {                                                \
        p.task0 = (int)t0;                                                                          \
        const dim3 g((unsigned)pl.KS, (unsigned)ntb, (unsigned)std::min<int64_t>(65535, ntasks - t0)); \
        if (kt && t0 == 0) hipExtLaunchKernelGGL(K, g, b, lds, s, kt->start, kt->stop, 0, p);      \
        else K<<<g, b, lds, s>>>(p);                                                                \
        const hipError_t e_ = hipGetLastError();                                                    \
        if (e_ != hipSuccess) return e_;                                                            \
    }                                                                                               \
    return hipSuccess;
#define QMM_MMA(T)                                                                                  \
    if (pl.cm == 8) { QMM_MMA_K(k_gemv_mma<T>) }                                                    \
    if (pl.cm == 16) { QMM_MMA_K(k_gemv_mma16<T>) }                                                 \
    QMM_MMA_K(k_gemv_mma32<T>)
        switch (type) {
            case QMM_TYPE_Q4_0: { QMM_MMA(QMM_TYPE_Q4_0) }
            case QMM_TYPE_Q8_0: { QMM_MMA(QMM_TYPE_Q8_0) }
            case QMM_TYPE_Q4_K: { QMM_MMA(QMM_TYPE_Q4_K) }
            case QMM_TYPE_IQ4_XS: { QMM_MMA(QMM_TYPE_IQ4_XS) }
            case QMM_TYPE_IQ4_NL: { QMM_MMA(QMM_TYPE_IQ4_NL) }
            case QMM_TYPE_Q6_K: { QMM_MMA(QMM_TYPE_Q6_K) }
            default: return hipErrorInvalidValue;
        }
#undef QMM_MMA
#undef QMM_MMA_K
    }
    if (pl.nc > kMaxTaskCols) return hipErrorInvalidValue;
    switch (type) {
        case QMM_TYPE_Q4_0:   return launch_t<QMM_TYPE_Q4_0>(p, pl.nc, nwg, s, kt);
        case QMM_TYPE_Q8_0:   return launch_t<QMM_TYPE_Q8_0>(p, pl.nc, nwg, s, kt);
        case QMM_TYPE_Q4_K:   return launch_t<QMM_TYPE_Q4_K>(p, pl.nc, nwg, s, kt);
        case QMM_TYPE_Q6_K:   return launch_t<QMM_TYPE_Q6_K>(p, pl.nc, nwg, s, kt);
        case QMM_TYPE_IQ4_XS: return launch_t<QMM_TYPE_IQ4_XS>(p, pl.nc, nwg, s, kt);
        case QMM_TYPE_Q5_K:   return launch_t<QMM_TYPE_Q5_K>(p, pl.nc, nwg, s, kt);
        case QMM_TYPE_IQ4_NL: return launch_t<QMM_TYPE_IQ4_NL>(p, pl.nc, nwg, s, kt);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
