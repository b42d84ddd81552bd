// k_gemv.hip - dequant-fused decode GEMV (N = 1..8 columns per task) on gfx950.
//
// Role of the reference's kernel_mul_mv_{q4_K,q6_K}_q8_1 (P01:3740-3921),
// kernel_mul_mv_q4_0_q8_1 (P02:6098-6220), kernel_mul_mv_iq4_xs_q8_1
// (P01:3457-3553) and the MUL_MAT_ID matvec (P01:3923-3964), redesigned for
// CDNA4 and for ggml-cpu's numerics instead of the reference's two-term q8_1:
//  * activations are the vec_dot type's codes (q8_0 or q8_K, made on the
//    device bit-exactly by k_quant.hip) staged per work-group in LDS, so the
//    integer dot of every (sub-)block equals ggml-cpu's exactly and only the
//    fp32 combine order differs;
//  * each lane streams 16-byte units of the weight planes (one wave load =
//    1 KB contiguous per row), unpacks nibbles / 6-bit codes / the IQ4
//    codebook in VGPRs and reduces with v_dot4_i32_i8;
//  * LPR lanes share one row (LPR = 64 for rows of >= 64 units), the partial
//    sums are reduced across them with lane shuffles at the end.
// A task is up to NC activation columns against one weight matrix; dense
// MUL_MAT derives its task from the grid, MUL_MAT_ID reads device-built tasks.
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
    int kc;                      // weights per LDS chunk
    int lpr_log2;                // lanes per row = 1 << lpr_log2
    int riw;                     // row iterations per wave
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
// part p: chunk c = p/2, bytes 16h..16h+15 (h = p%2) of the chunk's 32 code
// bytes: low nibbles are weights 64c+16h+[0,16) (sub-block 2c), high nibbles
// 64c+32+16h+[0,16) (sub-block 2c+1).
template <> struct GV<QMM_TYPE_Q4_K> {
    static constexpr int BLK = 256, UPB = 8, BS = 256, SS = 16;
    struct W { uint4 q, h; };
    __device__ static void load(W & w, const WView & v, int64_t blk, int part) {
        const uint8_t * b = v.p[0] + blk * 144;
        w.h = ld16_nt(b);
        w.q = ld16_nt(b + 16 + 16 * part);
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
        w.sc.x = ldg_nt(sp);
        w.sc.y = ldg_nt(sp + 1);
        w.d = ldg_nt(reinterpret_cast<const uint16_t *>(v.p[3]) + blk);
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
        w.h.x = ldg_nt(hp);
        w.h.y = ldg_nt(hp + 1);
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

// prefetch depth (items in flight per lane) by type
template <int TYPE> constexpr int depth() { return TYPE == QMM_TYPE_Q6_K ? 3 : 4; }

// Quantize columns [0, nc) of the activation chunk [k0, k0 + kcur) into LDS
// (codes, scales, sums), exactly as the stand-alone pre-pass does.
template <int NC, int BS, int SS>
__device__ void quantize_chunk(const GemvParams & p, const int64_t * s_col, int nc, int64_t k0, int kcur,
                               uint8_t * lds) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int8_t * codes = reinterpret_cast<int8_t *>(lds);
    float * ds = reinterpret_cast<float *>(lds + (size_t)NC * p.kc);
    int16_t * ss = reinterpret_cast<int16_t *>(lds + (size_t)NC * p.kc + (size_t)NC * (p.kc / BS) * 4);
    if constexpr (BS == 256) {
        const int nsb = kcur / 256;
        for (int it = wave; it < nc * nsb; it += kWaves) {          // one wave per super-block
            const int j = it / nsb, sb = it - j * nsb;
            const float * x = f32_col(p.src, s_col[j]) + k0 + sb * 256 + 4 * lane;
            float v[4] = { x[0], x[1], x[2], x[3] };
            float d;
            int bs;
            const uint32_t q = quant_q8_K_wave(v, lane, &d, &bs);
            *reinterpret_cast<uint32_t *>(codes + (size_t)j * p.kc + sb * 256 + 4 * lane) = q;
            if ((lane & 3) == 0) ss[j * (p.kc / SS) + sb * 16 + (lane >> 2)] = (int16_t)bs;
            if (lane == 0) ds[j * (p.kc / BS) + sb] = d;
        }
    } else {
        const int nb = kcur / 32;                                   // 8 lanes per block
        for (int it = tid >> 3; it < ((nc * nb + 7) & ~7); it += kThreads / 8) {
            const bool live = it < nc * nb;
            const int j = live ? it / nb : 0, b = live ? it - j * nb : 0, q4 = tid & 7;
            float v[4] = { 0.f, 0.f, 0.f, 0.f };
            if (live) {
                const float * x = f32_col(p.src, s_col[j]) + k0 + b * 32 + 4 * q4;
                v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
            }
            float d;
            int sm;
            const uint32_t q = quant_q8_0_lane(v, &d, &sm);
            if (live) {
                *reinterpret_cast<uint32_t *>(codes + (size_t)j * p.kc + b * 32 + 4 * q4) = q;
                if (q4 == 0) {
                    ds[j * (p.kc / BS) + b] = d;
                    ss[j * (p.kc / SS) + b] = (int16_t)sm;
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

// One work-group: rows [row0, row0 + 4 * riw * RG) of one task's matrix.
// Each lane streams its items (row iteration ri, unit iteration i) with
// depth() weight units in flight; at the end of every row the LPR lanes of
// the row reduce their partial sums, which accumulate per row in LDS across
// K chunks and are written once at the end.
template <int TYPE, int NC>
__global__ __launch_bounds__(kThreads) void k_gemv(GemvParams p) {
    using T = GV<TYPE>;
    constexpr int D = depth<TYPE>();
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int64_t s_col[NC];      // activation column ids
    __shared__ int64_t s_doff[NC];

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
        const int64_t b = blockIdx.y / p.tpb, tt = blockIdx.y % p.tpb;
        const int64_t i2 = b % p.ne12, i3 = b / p.ne12;
        mat = (int)((i2 / p.r2) + (i3 / p.r3) * p.ne02);
        const int64_t first = tt * NC;
        nc = (int)((p.ne11 - first) < NC ? (p.ne11 - first) : NC);
        if (threadIdx.x < NC && (int)threadIdx.x < nc) {
            const int64_t i1 = first + threadIdx.x;
            s_col[threadIdx.x] = b * p.ne11 + i1;
            s_doff[threadIdx.x] = i1 * p.d_nb1 + i2 * p.d_nb2 + i3 * p.d_nb3;
        }
    }
    if (mat < 0 || nc <= 0) return;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lprl = p.lpr_log2, LPR = 1 << lprl, RG = 64 >> lprl;
    const int rl = lane & (LPR - 1), rs = lane >> lprl;
    const int rows_wg = kWaves * p.riw * RG;
    const int64_t row0 = (int64_t)blockIdx.x * rows_wg;
    const int64_t bpr = p.w.bpr;
    const XL<NC, T::BS, T::SS> x{ lds, p.kc };
    const size_t xbytes = (size_t)NC * p.kc + (size_t)NC * (p.kc / T::BS) * 4 + (size_t)NC * (p.kc / T::SS) * 2;
    float * rowacc = reinterpret_cast<float *>(lds + ((xbytes + 15) & ~(size_t)15));   // [rows_wg][NC]

    for (int64_t k0 = 0; k0 < p.K; k0 += p.kc) {
        const int kcur = (int)((p.K - k0) < p.kc ? (p.K - k0) : p.kc);
        __syncthreads();
        if (p.fused) quantize_chunk<NC, T::BS, T::SS>(p, s_col, nc, k0, kcur, lds);
        else stage_chunk<NC, T::BS, T::SS>(p, s_col, nc, k0, kcur, lds);
        __syncthreads();

        const int nunits = (kcur / T::BLK) * T::UPB;
        const int upl = (nunits + LPR - 1) >> lprl;           // unit iterations per row
        const int nitems = p.riw * upl;
        const int64_t kblk0 = k0 / T::BLK;
        auto item = [&](int t, int64_t & blk, int & u, int & rloc) -> bool {
            const int ri = t / upl, i = t - ri * upl;
            rloc = (wave * p.riw + ri) * RG + rs;
            u = rl + (i << lprl);
            const int64_t row = row0 + rloc;
            blk = ((int64_t)mat * p.M + row) * bpr + kblk0 + u / T::UPB;
            return row < p.M && u < nunits;
        };
        typename T::W buf[D];
#pragma unroll
        for (int j = 0; j < D; ++j) {
            int64_t blk;
            int u, rloc;
            if (j < nitems && item(j, blk, u, rloc)) T::load(buf[j], p.w, blk, u % T::UPB);
        }
        float acc[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) acc[j] = 0.0f;
        for (int t0 = 0; t0 < nitems; t0 += D) {
#pragma unroll
            for (int j = 0; j < D; ++j) {
                const int t = t0 + j;
                if (t < nitems) {
                    const typename T::W cur = buf[j];
                    int64_t blk;
                    int u, rloc;
                    if (t + D < nitems && item(t + D, blk, u, rloc)) T::load(buf[j], p.w, blk, u % T::UPB);
                    const bool ok = item(t, blk, u, rloc);
                    if (ok) T::template dot<NC>(cur, u / T::UPB, u % T::UPB, x, nc, acc);
                    if ((t % upl) == upl - 1) {        // last unit iteration of a row (uniform)
#pragma unroll
                        for (int c = 0; c < NC; ++c) {
                            const float v = group_sum(acc[c], LPR);
                            acc[c] = 0.0f;
                            if (c < nc && rl == 0 && rloc < rows_wg) {
                                float & r = rowacc[rloc * NC + c];
                                r = (k0 == 0) ? v : r + v;
                            }
                        }
                    }
                }
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < rows_wg * nc; i += kThreads) {
        const int c = i / rows_wg, r = i - c * rows_wg;
        const int64_t row = row0 + r;
        if (row < p.M) p.dst[s_doff[c] + row] = rowacc[r * NC + c];
    }
}

template <int TYPE>
hipError_t launch_t(const GemvParams & p, int nc, int64_t rows_per_wg, int64_t ntasks, size_t lds_bytes, hipStream_t s) {
    const dim3 grid((unsigned)((p.M + rows_per_wg - 1) / rows_per_wg), (unsigned)ntasks);
    switch (nc) {
#define QMM_NC(N)                                                                                         \
    case N:                                                                                               \
        if (lds_bytes > 65536)                                                                            \
            (void)hipFuncSetAttribute((const void *)k_gemv<TYPE, N>, hipFuncAttributeMaxDynamicSharedMemorySize, \
                                      (int)lds_bytes);                                                    \
        k_gemv<TYPE, N><<<grid, kThreads, lds_bytes, s>>>(p);                                             \
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

}  // namespace

hipError_t launch_gemv_any(int type, const WView & w, int64_t M, int64_t K, const ActBuf * a, const F32Cols * src,
                           const GemvTask * tasks, int ntasks_max, const int32_t * ntasks_dev, int nc,
                           const GemvDense * dense, float * dst, hipStream_t s) {
    const TypeShape ts = type_shape(type);
    if (!ts.blk || nc < 1 || nc > kMaxTaskCols || K % ts.blk || (!a && !src)) return hipErrorInvalidValue;
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
    // lanes per row: enough to cover a row's units in one pass, at most a wave
    const int64_t units = (K / ts.blk) * ts.upb;
    int lprl = 0;
    while ((1 << lprl) < units && lprl < 6) ++lprl;
    p.lpr_log2 = lprl;
    const int RG = 64 >> lprl;
    // rows per wave: aim at ~1024 work-groups over all tasks
    int riw = env_int("QMM_GEMV_RIW", 0);
    if (riw <= 0) {
        const int64_t target = std::max<int64_t>(1, 1024 / ntasks);
        riw = (int)((M + (int64_t)kWaves * RG * target - 1) / ((int64_t)kWaves * RG * target));
        riw = std::max(1, std::min(riw, 16));
    }
    p.riw = riw;
    const int64_t rows_per_wg = (int64_t)kWaves * riw * RG;
    // LDS chunk: up to 48 KB of activations per work-group
    const double per_k = 1.0 + 4.0 / ts.bs + 2.0 / ts.ss;
    int64_t kc = (int64_t)(49152.0 / (nc * per_k));
    kc = kc / 256 * 256;
    if (kc >= K || kc <= 0) kc = K;
    p.kc = (int)kc;
    const size_t xbytes = (size_t)nc * kc + (size_t)nc * (kc / ts.bs) * 4 + (size_t)nc * (kc / ts.ss) * 2;
    const size_t lds_bytes = ((xbytes + 15) & ~(size_t)15) + (size_t)rows_per_wg * nc * 4;
    switch (type) {
        case QMM_TYPE_Q4_0:   return launch_t<QMM_TYPE_Q4_0>(p, nc, rows_per_wg, ntasks, lds_bytes, s);
        case QMM_TYPE_Q8_0:   return launch_t<QMM_TYPE_Q8_0>(p, nc, rows_per_wg, ntasks, lds_bytes, s);
        case QMM_TYPE_Q4_K:   return launch_t<QMM_TYPE_Q4_K>(p, nc, rows_per_wg, ntasks, lds_bytes, s);
        case QMM_TYPE_Q6_K:   return launch_t<QMM_TYPE_Q6_K>(p, nc, rows_per_wg, ntasks, lds_bytes, s);
        case QMM_TYPE_IQ4_XS: return launch_t<QMM_TYPE_IQ4_XS>(p, nc, rows_per_wg, ntasks, lds_bytes, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
