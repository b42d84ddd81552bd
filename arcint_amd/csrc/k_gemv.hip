// k_gemv.hip - dequant-fused decode GEMV (N = 1..8 columns per task) on gfx950.
//
// Role of the reference's kernel_mul_mv_{q4_K,q6_K}_q8_1 (P01:3740-3921),
// kernel_mul_mv_q4_0_q8_1 (P02:6098-6220), kernel_mul_mv_iq4_xs_q8_1
// (P01:3457-3553) and the MUL_MAT_ID matvec (P01:3923-3964), redesigned for
// CDNA4 and for ggml-cpu's numerics instead of the reference's two-term q8_1:
//  * activations are the vec_dot type's codes (q8_0 or q8_K, bit-exact with
//    ggml-cpu's from_float) staged per work-group in LDS, so the integer dot
//    of every (sub-)block equals ggml-cpu's exactly and only the fp32 combine
//    order differs;
//  * each lane streams 16-byte units of the weight planes (one wave load
//    instruction = 64 contiguous 16-byte units), unpacks nibbles / 6-bit
//    codes / the IQ4 codebook in VGPRs and reduces with v_dot4_i32_i8;
//  * LPR lanes share one row (LPR chosen per shape so that few lanes idle),
//    a wave covers RG = 64 / LPR rows at a time and walks row groups with a
//    grid stride; the weight loads run D units ahead of the arithmetic in a
//    register ring that crosses row boundaries, and the first D loads are in
//    flight before the work-group quantizes x into LDS;
//  * partial sums of a row are reduced across its LPR lanes with cross-lane
//    adds once per row and written straight to dst (accumulated across K
//    chunks when x does not fit LDS at once).
// A task is up to NC activation columns against one weight matrix; dense
// MUL_MAT derives its task from blockIdx.y, MUL_MAT_ID reads device-built
// task lists.
#include "qmm_device.h"

#include <algorithm>
#include <cstdlib>

namespace qmm {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

struct GemvParams {
    WView w;
    int64_t M, K;
    ActBuf a;                    // pre-quantized activations (fused == 0)
    F32Cols src;                 // f32 activations quantized in LDS (fused == 1)
    int fused;
    const GemvTask * tasks;      // list mode when non-null
    const int32_t * ntasks_dev;
    // dense mode: task y -> batch b = y / tpb, columns (y % tpb) * NC ...
    int64_t ne11, ne12, r2, r3, ne02, tpb;
    int64_t d_nb1, d_nb2, d_nb3; // dst strides in floats
    float * dst;
    int kc;                      // weights per LDS chunk (a multiple of 256, or K)
    int lpr_log2;                // lanes per row = 1 << lpr_log2
    int64_t ngroups;             // row groups of 64 / LPR rows
};

// activation chunk in LDS: NC columns of codes, then scales, then sums
template <int NC, int BS, int SS>
struct XL {
    const uint8_t * base;
    int kc;
    __device__ const int8_t * codes(int j) const { return reinterpret_cast<const int8_t *>(base) + (size_t)j * kc; }
    __device__ const float * d(int j) const {
        return reinterpret_cast<const float *>(base + (size_t)NC * kc) + (size_t)j * (kc / BS);
    }
    __device__ const int16_t * sums(int j) const {
        return reinterpret_cast<const int16_t *>(base + (size_t)NC * kc + (size_t)NC * (kc / BS) * 4) + (size_t)j * (kc / SS);
    }
};

__device__ __forceinline__ uint4 lds16(const int8_t * p) { return *reinterpret_cast<const uint4 *>(p); }

template <int TYPE> struct GV;

// ---- Q4_0: unit = one 32-weight block (16 B codes + fp16 d) ---------------
template <> struct GV<QMM_TYPE_Q4_0> {
    static constexpr int BLK = 32, UPB = 1, BS = 32, SS = 32;
    struct W { uint4 q; uint32_t d; };
    __device__ static void load(W & w, const WView & v, int64_t blk, int) {
        w.q = ld16_nt(v.p[0] + blk * 16);
        w.d = ldg_nt(reinterpret_cast<const uint16_t *>(v.p[1]) + blk);
    }
    template <int NC>
    __device__ static void dot(const W & w, int kb, int, const XL<NC, BS, SS> & x, int nc, float * acc) {
        const float dw = h2f(w.d);
        const uint32_t m = 0x0F0F0F0Fu;
        const uint32_t l0 = w.q.x & m, l1 = w.q.y & m, l2 = w.q.z & m, l3 = w.q.w & m;
        const uint32_t h0 = (w.q.x >> 4) & m, h1 = (w.q.y >> 4) & m, h2 = (w.q.z >> 4) & m, h3 = (w.q.w >> 4) & m;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            if (j < nc) {
                const int8_t * xc = x.codes(j) + kb * 32;
                const uint4 a = lds16(xc), b = lds16(xc + 16);
                int s = dot4(l0, a.x, dot4(l1, a.y, dot4(l2, a.z, dot4(l3, a.w, 0))));
                s = dot4(h0, b.x, dot4(h1, b.y, dot4(h2, b.z, dot4(h3, b.w, s))));
                s -= 8 * (int)x.sums(j)[kb];             // codes are q, the weight is q - 8
                acc[j] += (float)s * (dw * x.d(j)[kb]);
            }
        }
    }
};

// ---- Q8_0: unit = one 32-weight block (32 B codes + fp16 d) ---------------
template <> struct GV<QMM_TYPE_Q8_0> {
    static constexpr int BLK = 32, UPB = 1, BS = 32, SS = 32;
    struct W { uint4 q0, q1; uint32_t d; };
    __device__ static void load(W & w, const WView & v, int64_t blk, int) {
        w.q0 = ld16_nt(v.p[0] + blk * 32);
        w.q1 = ld16_nt(v.p[0] + blk * 32 + 16);
        w.d = ldg_nt(reinterpret_cast<const uint16_t *>(v.p[1]) + blk);
    }
    template <int NC>
    __device__ static void dot(const W & w, int kb, int, const XL<NC, BS, SS> & x, int nc, float * acc) {
        const float dw = h2f(w.d);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            if (j < nc) {
                const int8_t * xc = x.codes(j) + kb * 32;
                const uint4 a = lds16(xc), b = lds16(xc + 16);
                int s = dot4(w.q0.x, a.x, dot4(w.q0.y, a.y, dot4(w.q0.z, a.z, dot4(w.q0.w, a.w, 0))));
                s = dot4(w.q1.x, b.x, dot4(w.q1.y, b.y, dot4(w.q1.z, b.z, dot4(w.q1.w, b.w, s))));
                acc[j] += (float)s * (dw * x.d(j)[kb]);
            }
        }
    }
};

// ---- Q4_K: unit = 16 B of codes (part p of 8) + the 16 B block header -----
// Planes: codes qs[128] per block, header {d, dmin, scales[12]} per block.
// part p: chunk c = p/2, bytes 16h..16h+15 (h = p%2) of the chunk's 32 code
// bytes: low nibbles are weights 64c+16h+[0,16) (sub-block 2c), high nibbles
// 64c+32+16h+[0,16) (sub-block 2c+1).
template <> struct GV<QMM_TYPE_Q4_K> {
    static constexpr int BLK = 256, UPB = 8, BS = 256, SS = 16;
    struct W { uint4 q, h; };
    __device__ static void load(W & w, const WView & v, int64_t blk, int part) {
        w.q = ld16_nt(v.p[0] + blk * 128 + 16 * part);
        w.h = ld16(v.p[1] + blk * 16);            // shared by the block's 8 lanes: keep it cached
    }
    template <int NC>
    __device__ static void dot(const W & w, int kb, int part, const XL<NC, BS, SS> & x, int nc, float * acc) {
        const int c = part >> 1, hh = part & 1;
        // 6-bit scales / mins (get_scale_min_k4, P01:2164-2176), four per dword
        const uint32_t s0 = w.h.y, s1 = w.h.z, s2 = w.h.w;
        const uint32_t scd = c < 2 ? (s0 & 0x3f3f3f3fu) : ((s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u));
        const uint32_t mnd = c < 2 ? (s1 & 0x3f3f3f3fu) : (((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u));
        const int sh = (c & 1) * 16;
        const int sc_a = (scd >> sh) & 0xff, sc_b = (scd >> (sh + 8)) & 0xff;
        const int m_a = (mnd >> sh) & 0xff, m_b = (mnd >> (sh + 8)) & 0xff;
        const float d = h2f(w.h.x), dmin = h2f(w.h.x >> 16);
        const uint32_t m = 0x0F0F0F0Fu;
        const uint32_t l0 = w.q.x & m, l1 = w.q.y & m, l2 = w.q.z & m, l3 = w.q.w & m;
        const uint32_t h0 = (w.q.x >> 4) & m, h1 = (w.q.y >> 4) & m, h2 = (w.q.z >> 4) & m, h3 = (w.q.w >> 4) & m;
        const int ko = kb * 256 + 64 * c + 16 * hh;
        const int bo = kb * 16 + 4 * c + hh;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            if (j < nc) {
                const int8_t * xc = x.codes(j) + ko;
                const uint4 a = lds16(xc), b = lds16(xc + 32);
                const int sa = dot4(l0, a.x, dot4(l1, a.y, dot4(l2, a.z, dot4(l3, a.w, 0))));
                const int sb = dot4(h0, b.x, dot4(h1, b.y, dot4(h2, b.z, dot4(h3, b.w, 0))));
                const int16_t * bs = x.sums(j) + bo;
                const int isc = sc_a * sa + sc_b * sb;
                const int imn = m_a * (int)bs[0] + m_b * (int)bs[2];
                acc[j] += x.d(j)[kb] * (d * (float)isc - dmin * (float)imn);
            }
        }
    }
};

// ---- Q6_K: unit = 64 weights (half n, l0 = 16 * (u & 1)) ------------------
// codes 128n + 32g + l0 + [0,16) for g = 0..3 from ql[64n+l0], ql[64n+32+l0]
// (low nibbles g = 0, 1; high g = 2, 3) and qh[32n+l0] bits 2g..2g+1; scale
// of group g is scales[8n + 2g + (u & 1)].
template <> struct GV<QMM_TYPE_Q6_K> {
    static constexpr int BLK = 256, UPB = 4, BS = 256, SS = 16;
    struct W { uint4 qa, qb, qh; uint2 sc; uint32_t d; };
    __device__ static void load(W & w, const WView & v, int64_t blk, int u) {
        const int n = u >> 1, l0 = 16 * (u & 1);
        w.qa = ld16_nt(v.p[0] + blk * 128 + 64 * n + l0);
        w.qb = ld16_nt(v.p[0] + blk * 128 + 64 * n + 32 + l0);
        w.qh = ld16_nt(v.p[1] + blk * 64 + 32 * n + l0);
        const uint32_t * sp = reinterpret_cast<const uint32_t *>(v.p[2] + blk * 16 + 8 * n);
        w.sc.x = sp[0];
        w.sc.y = sp[1];
        w.d = reinterpret_cast<const uint16_t *>(v.p[3])[blk];
    }
    __device__ static void codes(const W & w, int g, uint32_t o[4]) {
        const uint32_t m = 0x0F0F0F0Fu, mh = 0x30303030u;
        const uint32_t ql[4] = { (g & 1) ? w.qb.x : w.qa.x, (g & 1) ? w.qb.y : w.qa.y,
                                 (g & 1) ? w.qb.z : w.qa.z, (g & 1) ? w.qb.w : w.qa.w };
        const uint32_t qh[4] = { w.qh.x, w.qh.y, w.qh.z, w.qh.w };
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = g < 2 ? (ql[i] & m) : ((ql[i] >> 4) & m);
            const uint32_t hi = g == 0 ? (qh[i] << 4) : g == 1 ? (qh[i] << 2) : g == 2 ? qh[i] : (qh[i] >> 2);
            o[i] = lo | (hi & mh);
        }
    }
    template <int NC>
    __device__ static void dot(const W & w, int kb, int u, const XL<NC, BS, SS> & x, int nc, float * acc) {
        const int n = u >> 1, p = u & 1, l0 = 16 * p;
        const float dw = h2f(w.d);
        uint32_t cg[4][4];
        int scg[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            codes(w, g, cg[g]);
            const int byte = 2 * g + p;
            const uint32_t sw = byte < 4 ? w.sc.x : w.sc.y;
            scg[g] = (int)(int8_t)((sw >> (8 * (byte & 3))) & 0xff);
        }
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            if (j < nc) {
                int isum = 0;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int8_t * xc = x.codes(j) + kb * 256 + 128 * n + 32 * g + l0;
                    const uint4 a = lds16(xc);
                    int s = dot4(cg[g][0], a.x, dot4(cg[g][1], a.y, dot4(cg[g][2], a.z, dot4(cg[g][3], a.w, 0))));
                    s -= 32 * (int)x.sums(j)[kb * 16 + 8 * n + 2 * g + p];   // codes are q, the weight q - 32
                    isum += scg[g] * s;
                }
                acc[j] += (float)isum * (dw * x.d(j)[kb]);
            }
        }
    }
};

// ---- IQ4_XS: unit = one 32-weight sub-block ib (16 B codes + 8 B header) --
template <> struct GV<QMM_TYPE_IQ4_XS> {
    static constexpr int BLK = 256, UPB = 8, BS = 256, SS = 16;
    struct W { uint4 q; uint2 h; };
    __device__ static void load(W & w, const WView & v, int64_t blk, int ib) {
        w.q = ld16_nt(v.p[0] + blk * 128 + 16 * ib);
        const uint32_t * hp = reinterpret_cast<const uint32_t *>(v.p[1] + blk * 8);
        w.h.x = hp[0];
        w.h.y = hp[1];
    }
    template <int NC>
    __device__ static void dot(const W & w, int kb, int ib, const XL<NC, BS, SS> & x, int nc, float * acc) {
        const float dw = h2f(w.h.x);
        const uint32_t sh = w.h.x >> 16;
        const int ls = (int)(((w.h.y >> (4 * ib)) & 0xF) | (((sh >> (2 * ib)) & 3) << 4));
        const float dls = (float)(ls - 32);
        const uint32_t q[4] = { w.q.x, w.q.y, w.q.z, w.q.w };
        uint32_t vl[4], vh[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            vl[i] = iq4_lookup(q[i] & 0x0F0F0F0Fu);
            vh[i] = iq4_lookup((q[i] >> 4) & 0x0F0F0F0Fu);
        }
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            if (j < nc) {
                const int8_t * xc = x.codes(j) + kb * 256 + 32 * ib;
                const uint4 a = lds16(xc), b = lds16(xc + 16);
                int s = dot4(vl[0], a.x, dot4(vl[1], a.y, dot4(vl[2], a.z, dot4(vl[3], a.w, 0))));
                s = dot4(vh[0], b.x, dot4(vh[1], b.y, dot4(vh[2], b.z, dot4(vh[3], b.w, s))));
                acc[j] += ((dw * x.d(j)[kb]) * dls) * (float)s;
            }
        }
    }
};

// weight units in flight per lane, by type (register budget: D * sizeof(W))
template <int TYPE> constexpr int depth() {
    return TYPE == QMM_TYPE_Q6_K ? 4 : (TYPE == QMM_TYPE_Q8_0 || TYPE == QMM_TYPE_Q4_K) ? 6 : 8;
}

// Quantize columns [0, nc) of the activation chunk [k0, k0 + kcur) into LDS
// (codes, scales, sums), bit-identical to the stand-alone pre-pass.  The x
// loads of QB items are issued together before any of them is used, so the
// prologue pays about one L2 round trip per QB items rather than one each.
template <int NC, int BS, int SS>
__device__ void quantize_chunk(const GemvParams & p, const float * const * s_x, int nc, int64_t k0, int kcur,
                               uint8_t * lds) {
    constexpr int QB = 4;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int8_t * codes = reinterpret_cast<int8_t *>(lds);
    float * ds = reinterpret_cast<float *>(lds + (size_t)NC * p.kc);
    int16_t * ss = reinterpret_cast<int16_t *>(lds + (size_t)NC * p.kc + (size_t)NC * (p.kc / BS) * 4);
    if constexpr (BS == 256) {
        // one wave per 256-weight super-block, 4 weights per lane
        const int nsb = kcur / 256, total = nc * nsb;
        for (int it0 = wave; it0 < total; it0 += kWaves * QB) {
            float v[QB][4];
#pragma unroll
            for (int q = 0; q < QB; ++q) {
                const int it = it0 + q * kWaves;
                if (it < total) {
                    const int j = it / nsb, sb = it - j * nsb;
                    const float * x = s_x[j] + k0 + sb * 256 + 4 * lane;
                    v[q][0] = x[0]; v[q][1] = x[1]; v[q][2] = x[2]; v[q][3] = x[3];
                }
            }
#pragma unroll
            for (int q = 0; q < QB; ++q) {
                const int it = it0 + q * kWaves;
                if (it < total) {                                  // uniform per wave
                    const int j = it / nsb, sb = it - j * nsb;
                    float d;
                    int bs;
                    const uint32_t c = quant_q8_K_wave(v[q], lane, &d, &bs);
                    *reinterpret_cast<uint32_t *>(codes + (size_t)j * p.kc + sb * 256 + 4 * lane) = c;
                    if ((lane & 3) == 0) ss[j * (p.kc / SS) + sb * 16 + (lane >> 2)] = (int16_t)bs;
                    if (lane == 0) ds[j * (p.kc / BS) + sb] = d;
                }
            }
        }
    } else {
        // 8 lanes per 32-weight block, 4 weights per lane; the loop bounds are
        // uniform over the work-group so every lane takes part in the
        // 8-lane reductions
        const int nb = kcur / 32, total = nc * nb, q4 = tid & 7;
        for (int it0 = 0; it0 < total; it0 += (kThreads / 8) * QB) {
            float v[QB][4];
#pragma unroll
            for (int q = 0; q < QB; ++q) {
                const int it = it0 + q * (kThreads / 8) + (tid >> 3);
                v[q][0] = v[q][1] = v[q][2] = v[q][3] = 0.0f;
                if (it < total) {
                    const int j = it / nb, b = it - j * nb;
                    const float * x = s_x[j] + k0 + b * 32 + 4 * q4;
                    v[q][0] = x[0]; v[q][1] = x[1]; v[q][2] = x[2]; v[q][3] = x[3];
                }
            }
#pragma unroll
            for (int q = 0; q < QB; ++q) {
                const int it = it0 + q * (kThreads / 8) + (tid >> 3);
                float d;
                int sm;
                const uint32_t c = quant_q8_0_lane(v[q], &d, &sm);
                if (it < total) {
                    const int j = it / nb, b = it - j * nb;
                    *reinterpret_cast<uint32_t *>(codes + (size_t)j * p.kc + b * 32 + 4 * q4) = c;
                    if (q4 == 0) {
                        ds[j * (p.kc / BS) + b] = d;
                        ss[j * (p.kc / SS) + b] = (int16_t)sm;
                    }
                }
            }
        }
    }
}

// copy pre-quantized columns of the chunk into LDS
template <int NC, int BS, int SS>
__device__ void stage_chunk(const GemvParams & p, const int64_t * s_col, int nc, int64_t k0, int kcur, uint8_t * lds) {
    const int tid = threadIdx.x;
    const int n16 = kcur / 16;
    for (int i = tid; i < nc * n16; i += kThreads) {
        const int j = i / n16, o = (i - j * n16) * 16;
        *reinterpret_cast<uint4 *>(lds + (size_t)j * p.kc + o) =
            *reinterpret_cast<const uint4 *>(p.a.codes + s_col[j] * p.K + k0 + o);
    }
    const int nd = kcur / BS, ns = kcur / SS;
    float * ld = reinterpret_cast<float *>(lds + (size_t)NC * p.kc);
    int16_t * ls = reinterpret_cast<int16_t *>(lds + (size_t)NC * p.kc + (size_t)NC * (p.kc / BS) * 4);
    for (int i = tid; i < nc * nd; i += kThreads) {
        const int j = i / nd, o = i - j * nd;
        ld[j * (p.kc / BS) + o] = p.a.d[s_col[j] * (p.K / BS) + k0 / BS + o];
    }
    for (int i = tid; i < nc * ns; i += kThreads) {
        const int j = i / ns, o = i - j * ns;
        ls[j * (p.kc / SS) + o] = p.a.sums[s_col[j] * (p.K / SS) + k0 / SS + o];
    }
}

// One work-group: waves blockIdx.x * 4 + w walk row groups g, g + stride, ...
// of one task's matrix.  Lane (rs, rl) handles row g * RG + rs and units
// rl + LPR * i (i < UI) of it.  Items (g, i) are streamed through a D-deep
// register ring: item t is used from buf[t % D], then buf[t % D] is refilled
// with item t + D.  Every ring load is issued unconditionally (an item past
// the end loads the matrix's first block and is not used), so the number of
// loads in flight is static and each use waits only for its own load rather
// than for all of them.  MULTI: x spans several LDS chunks and the partial
// sums of later chunks are added to dst.
template <int TYPE, int NC, bool MULTI>
__global__ __launch_bounds__(kThreads) void k_gemv(GemvParams p) {
    using T = GV<TYPE>;
    using W = typename T::W;
    constexpr int D = depth<TYPE>();
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int64_t s_col[NC];      // activation column ids
    __shared__ int64_t s_doff[NC];     // float offset of dst row 0 per column
    __shared__ const float * s_x[NC];  // f32 activation columns (fused mode)

    // task decode; every count here fits 32 bits, so no 64-bit divisions
    int mat, nc;
    if (p.tasks) {
        if (p.ntasks_dev && (int)blockIdx.y >= *p.ntasks_dev) return;
        const GemvTask & t = p.tasks[blockIdx.y];
        mat = t.mat;
        nc = t.ncols;
        if (threadIdx.x < NC && (int)threadIdx.x < nc) {
            s_col[threadIdx.x] = t.col[threadIdx.x];
            s_doff[threadIdx.x] = t.dst_off[threadIdx.x];
        }
    } else {
        const uint32_t y = blockIdx.y, tpb = (uint32_t)p.tpb, ne12 = (uint32_t)p.ne12;
        const uint32_t b = y / tpb, tt = y - b * tpb;
        const uint32_t i3 = b / ne12, i2 = b - i3 * ne12;
        mat = (int)(i2 / (uint32_t)p.r2 + (i3 / (uint32_t)p.r3) * (uint32_t)p.ne02);
        const int64_t first = (int64_t)tt * NC;
        nc = (int)((p.ne11 - first) < NC ? (p.ne11 - first) : NC);
        if (threadIdx.x < NC && (int)threadIdx.x < nc) {
            const int64_t i1 = first + threadIdx.x;
            s_col[threadIdx.x] = (int64_t)b * p.ne11 + i1;
            s_doff[threadIdx.x] = i1 * p.d_nb1 + (int64_t)i2 * p.d_nb2 + (int64_t)i3 * p.d_nb3;
        }
    }
    if (mat < 0 || nc <= 0) return;    // uniform over the work-group
    if (p.fused && threadIdx.x < NC && (int)threadIdx.x < nc) s_x[threadIdx.x] = f32_col(p.src, s_col[threadIdx.x]);
    __syncthreads();                   // s_col, s_doff, s_x

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lprl = p.lpr_log2, LPR = 1 << lprl, RG = 64 >> lprl;
    const int rl = lane & (LPR - 1), rs = lane >> lprl;
    const int64_t g0 = (int64_t)blockIdx.x * kWaves + wave, gs = (int64_t)gridDim.x * kWaves;
    const int64_t ngroups = p.ngroups, M = p.M, bpr = p.w.bpr;
    const int64_t ngw = g0 < ngroups ? (int64_t)((uint32_t)(ngroups - 1 - g0) / (uint32_t)gs) + 1 : 0;   // row groups of this wave
    const int64_t row_step = gs * RG, blk_step = row_step * bpr;
    const XL<NC, T::BS, T::SS> x{ lds, p.kc };

    for (int64_t k0 = 0; k0 < p.K; k0 += p.kc) {
        const int kcur = (int)((p.K - k0) < p.kc ? (p.K - k0) : p.kc);
        const int nunits = (kcur / T::BLK) * T::UPB;
        const int UI = (nunits + LPR - 1) >> lprl;            // unit iterations per row
        const int nitems = (int)(ngw * UI);
        const int64_t blk0 = (int64_t)mat * M * bpr + k0 / T::BLK;   // (matrix, row 0, chunk start)

        // load cursor: row lrow (block lblk of its unit 0), unit iteration li
        int64_t lrow = g0 * RG + rs, lblk = blk0 + lrow * bpr;
        int li = 0;
        auto issue = [&](W & w) {
            const int u = rl + (li << lprl);
            const bool ok = lrow < M && u < nunits;
            T::load(w, p.w, ok ? lblk + u / T::UPB : blk0, ok ? u % T::UPB : 0);
            const bool wrap = ++li == UI;
            li = wrap ? 0 : li;
            lrow += wrap ? row_step : 0;
            lblk += wrap ? blk_step : 0;
        };
        W buf[D];
#pragma unroll
        for (int j = 0; j < D; ++j) issue(buf[j]);

        if (k0 > 0) __syncthreads();       // the previous chunk's LDS reads are done
        if (p.fused) quantize_chunk<NC, T::BS, T::SS>(p, s_x, nc, k0, kcur, lds);
        else stage_chunk<NC, T::BS, T::SS>(p, s_col, nc, k0, kcur, lds);
        __syncthreads();

        int64_t crow = g0 * RG + rs;
        int ci = 0;
        float acc[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) acc[j] = 0.0f;
        for (int t0 = 0; t0 < nitems; t0 += D) {
#pragma unroll
            for (int j = 0; j < D; ++j) {
                if (t0 + j < nitems) {             // uniform per wave
                    const int u = rl + (ci << lprl);
                    if (crow < M && u < nunits) T::template dot<NC>(buf[j], u / T::UPB, u % T::UPB, x, nc, acc);
                    if (++ci == UI) {              // the row is complete (uniform)
                        ci = 0;
#pragma unroll
                        for (int c = 0; c < NC; ++c) {
                            const float v = group_sum(acc[c], lprl);
                            acc[c] = 0.0f;
                            if (c < nc && rl == 0 && crow < M) {
                                float * o = p.dst + s_doff[c] + crow;
                                if constexpr (MULTI) *o = (k0 == 0) ? v : *o + v;
                                else *o = v;
                            }
                        }
                        crow += row_step;
                    }
                }
                issue(buf[j]);
            }
        }
    }
}

template <int TYPE, bool MULTI>
hipError_t launch_t(const GemvParams & p, int nc, int64_t nwg, int64_t ntasks, size_t lds_bytes, hipStream_t s) {
    const dim3 grid((unsigned)nwg, (unsigned)ntasks);
    switch (nc) {
#define QMM_NC(N)                                                                                         \
    case N:                                                                                               \
        if (lds_bytes > 65536)                                                                            \
            (void)hipFuncSetAttribute((const void *)k_gemv<TYPE, N, MULTI>,                               \
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);        \
        k_gemv<TYPE, N, MULTI><<<grid, kThreads, lds_bytes, s>>>(p);                                      \
        break;
        QMM_NC(1) QMM_NC(2) QMM_NC(3) QMM_NC(4) QMM_NC(5) QMM_NC(6) QMM_NC(7) QMM_NC(8)
#undef QMM_NC
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

struct TypeShape { int blk, upb, bs, ss; };
TypeShape type_shape(int type) {
    switch (type) {
        case QMM_TYPE_Q4_0:   return { 32, 1, 32, 32 };
        case QMM_TYPE_Q8_0:   return { 32, 1, 32, 32 };
        case QMM_TYPE_Q4_K:   return { 256, 8, 256, 16 };
        case QMM_TYPE_Q6_K:   return { 256, 4, 256, 16 };
        case QMM_TYPE_IQ4_XS: return { 256, 8, 256, 16 };
        default:              return { 0, 0, 0, 0 };
    }
}

int env_int(const char * name, int dflt) {
    const char * e = getenv(name);
    return e ? atoi(e) : dflt;
}

// lanes per row: the widest (fewest rows per wave) that keeps >= 90 % of the
// lanes busy on a row's units, else the one that idles the fewest lanes
int pick_lpr_log2(int64_t units) {
    int best = 6;
    double best_eff = -1.0;
    for (int l = 6; l >= 2; --l) {
        const int64_t lpr = 1 << l;
        const int64_t ui = (units + lpr - 1) / lpr;
        const double eff = (double)units / (double)(ui * lpr);
        if (eff >= 0.9) return l;
        if (eff > best_eff + 1e-9) { best_eff = eff; best = l; }
    }
    return best;
}

}  // namespace

hipError_t launch_gemv_any(int type, const WView & w, int64_t M, int64_t K, const ActBuf * a, const F32Cols * src,
                           const GemvTask * tasks, int ntasks_max, const int32_t * ntasks_dev, int nc,
                           const GemvDense * dense, float * dst, hipStream_t s) {
    const TypeShape ts = type_shape(type);
    if (!ts.blk || nc < 1 || nc > kMaxTaskCols || K % ts.blk || (!a && !src) || M <= 0) return hipErrorInvalidValue;
    GemvParams p{};
    p.w = w;
    p.M = M;
    p.K = K;
    if (a) p.a = *a;
    if (src) p.src = *src;
    p.fused = a ? 0 : 1;
    p.tasks = tasks;
    p.ntasks_dev = ntasks_dev;
    p.dst = dst;
    int64_t ntasks = ntasks_max;
    if (!tasks) {
        p.ne11 = dense->ne11;
        p.ne12 = dense->ne12;
        p.r2 = dense->r2;
        p.r3 = dense->r3;
        p.ne02 = dense->ne02;
        p.tpb = (dense->ne11 + nc - 1) / nc;
        p.d_nb1 = dense->d_nb1;
        p.d_nb2 = dense->d_nb2;
        p.d_nb3 = dense->d_nb3;
        ntasks = p.tpb * dense->ne12 * dense->ne13;
    }
    if (ntasks <= 0) return hipSuccess;
    if (ntasks > 65535) return hipErrorInvalidValue;
    // LDS chunk of x: up to ~40 KB per work-group (several work-groups per CU)
    const int lds_budget = env_int("QMM_GEMV_LDS", 40960);
    const double per_k = 1.0 + 4.0 / ts.bs + 2.0 / ts.ss;
    int64_t kc = (int64_t)((double)lds_budget / (nc * per_k));
    kc = kc / 256 * 256;
    if (kc >= K || kc <= 0) kc = K;
    p.kc = (int)kc;
    const int64_t units = (kc / ts.blk) * ts.upb;
    const int lprl = env_int("QMM_GEMV_LPR", 0) > 0 ? std::min(6, std::max(0, env_int("QMM_GEMV_LPR", 0))) : pick_lpr_log2(units);
    p.lpr_log2 = lprl;
    const int RG = 64 >> lprl;
    p.ngroups = (M + RG - 1) / RG;
    // work-groups per task: ~target over all tasks, no more than row groups
    const int64_t target = std::max(1, env_int("QMM_GEMV_WG", 1024));
    int64_t nwg = std::max<int64_t>(1, target / ntasks);
    nwg = std::min<int64_t>(nwg, (p.ngroups + kWaves - 1) / kWaves);
    const size_t lds_bytes = (size_t)nc * kc + (size_t)nc * (kc / ts.bs) * 4 + (size_t)nc * (kc / ts.ss) * 2;
    const bool multi = kc < K;
#define QMM_T(TY) return multi ? launch_t<TY, true>(p, nc, nwg, ntasks, lds_bytes, s) \
                               : launch_t<TY, false>(p, nc, nwg, ntasks, lds_bytes, s)
    switch (type) {
        case QMM_TYPE_Q4_0:   QMM_T(QMM_TYPE_Q4_0);
        case QMM_TYPE_Q8_0:   QMM_T(QMM_TYPE_Q8_0);
        case QMM_TYPE_Q4_K:   QMM_T(QMM_TYPE_Q4_K);
        case QMM_TYPE_Q6_K:   QMM_T(QMM_TYPE_Q6_K);
        case QMM_TYPE_IQ4_XS: QMM_T(QMM_TYPE_IQ4_XS);
        default: return hipErrorInvalidValue;
    }
#undef QMM_T
}

}  // namespace qmm
