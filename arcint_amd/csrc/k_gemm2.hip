// k_gemm2.hip - prefill GEMM (N >= 16 columns) for the five weight types on
// gfx950 v_mfma_i32_32x32x32_i8.
//
// Role of the reference's prefill GEMMs (the int8 kernel_mul_mm_kq2d_q4_0_i8,
// P0099:377-455, and kernel_mul_mm_kq2d_q4_K_i8, P01:1919-2024, and the fp16
// tile kernels kernel_mul_mm_{q6_K,iq4_xs,q8_0}_f16, P01:2317-2406,
// P02:4359-4384), redesigned for CDNA4 and for ggml-cpu's numerics:
//  * a work-group (8 waves) owns 128 weight rows (two 64-row tiles of the
//    weight image) x BN activation columns (BN = 128 or 64) and walks K in
//    stages of 128 (half a group).  Per stage it stages in LDS the activation
//    codes of its columns (a padded pitch spreads the columns over the banks),
//    its two tiles' weights unpacked into MFMA operands (once per work-group,
//    not once per wave) and the scales; the data of a stage is fetched two
//    stages ahead into registers and stored at the end of the stage before;
//  * a wave computes 64 rows x 32 columns as 2 MFMA tiles of 32 x 32, one
//    32-weight (sub-)block per MFMA.  Both operands place k in [16h, 16h + 16)
//    of the block in lane half h, so the int32 result is the block's exact
//    integer dot, as in ggml_vec_dot_*.  With BN = 64 two waves share each
//    tile, one taking blocks 0 and 2 of every stage and the other blocks 1
//    and 3, and their sums meet in LDS at the end (no atomics);
//  * Q4_0 / Q8_0: the weight operand is q - 8 / q.  The MFMA adds the block's dot i to
//    the bits of the float 12582912 (= 1.5 * 2^23), so fma(result, d_w,
//    -12582912 d_w) is i * d_w rounded once (12582912 d_w is exact), and
//    acc += d_x * that: two VALU ops per output and block;
//  * Q4_K: the 6-bit sub-block scale sc = 8 sh + sl is folded into two int8
//    operands q * sh and q * sl (a packed 16-bit multiply scales 4 codes at
//    once; every product is < 128), so the scale part of a super-block
//    accumulates inside the MFMA in int32.  The min term sum_j m_j bsum_j
//    takes two MFMAs per super-block: the activation sub-block sums split as
//    bsum = 64 bh + bl (bh in [-64, 63], bl in [0, 63]) against the 8 mins;
//  * IQ4_XS (codebook values, 6-bit scale per 32) and Q6_K (q - 32, int8
//    scale per 16): the scaled weights do not fit int8, so each (sub-)block
//    dot comes from a fresh MFMA and is multiplied by its integer scale into
//    an int32 sum on the VALU (Q6_K: one MFMA per 16-weight half, the other
//    half's operand zero); the float combine runs once per super-block;
//  * work-groups are numbered so that those sharing weight rows land on the
//    same XCD.  Small products split K over KS work-groups that add their
//    partial sums to dst (zeroed by the activation pre-pass) atomically.
// MFMA output layout: lane l holds D[8 (r/4) + 4 (l/32) + r%4][l % 32] in
// accumulator register r.
#include "qmm_device.h"

#include <hip/hip_ext.h>

#include <algorithm>
#include <cstdlib>

namespace qmm {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kT = 512;                  // threads per work-group (8 waves)
constexpr int kSK = 128;                 // k per stage
constexpr int kAP = kSK + 16;            // LDS pitch of one column's codes
constexpr int kMagic = 0x4B400000;       // float 12582912: its bits + i are the float 12582912 + i, |i| < 2^22

// LDS stage layout (bytes):
//   A  [col BN][kAP]                                 activation codes
//   Q4_0  B  [tile 2][block 4][h 2][row 64] x 16 B    q - 8
//         W  [tile 2][block 4][row 64] f32            d_w
//         X  [block 4][col BN] f32                    d_x
//   Q4_K  B  [tile 2][sub 4][h 2][hi/lo 2][row 64] x 16 B   q * sh, q * sl
//         W  [tile 2][row 64] x 16 B                  the super-block's 8 mins, then 8 zero bytes
//   Q5_K  as Q4_K with (q - 16) * sh, (q - 16) * sl, and the 8 scales after the mins (the
//         16 sum_j sc_j bsum_j that q - 16 takes off comes back from one more MFMA)
//            [tile 2][row 64] float2                  (d, dmin)
//         X  [col BN] f32                             d_x of the super-block
//         S  [col BN] x 16 B                          bh[8], bl[8] of the super-block
//   IQ4_XS, Q6_K (integer sub-block scales)
//         B  [tile 2][block 4][h 2][row 64] x 16 B    codebook value / q - 32
//         W  [tile 2][block 4][h 2][row 64] i32        ls - 32 (IQ4_XS: h = 0) / the 16-weight scale (Q6_K)
//            [tile 2][row 64] f32                     d
//         X  [col BN] f32                             d_x of the super-block
template <int TYPE, int BN> struct Lay {
    static constexpr bool KQ = TYPE == QMM_TYPE_Q4_K || TYPE == QMM_TYPE_Q5_K;
    static constexpr bool IS = TYPE == QMM_TYPE_IQ4_XS || TYPE == QMM_TYPE_Q6_K;
    static constexpr int A = BN * kAP;
    static constexpr int B = KQ ? 2 * 4 * 2 * 2 * kChunk : 2 * 4 * 2 * kChunk;
    static constexpr int W = KQ ? 2 * 64 * 16 + 2 * 64 * 8 : IS ? 2 * 4 * 2 * 64 * 4 + 2 * 64 * 4 : 2 * 4 * 64 * 4;
    static constexpr int X = (KQ || IS) ? BN * 4 : 4 * BN * 4;
    static constexpr int S = KQ ? BN * 16 : 0;
    static constexpr int oB = A, oW = oB + B, oX = oW + W, oS = oX + X;
    static constexpr int stage = oS + S;
};

struct G2Params {
    WView w;
    const int8_t * xc;                   // activation codes [col][ldk]
    int64_t ldk;
    const float * dT;                    // activation scales [block][ldT]
    int64_t ldT;
    const int8_t * bsp;                  // q8_K: split sub-block sums [super-block][ldT] x 16 B
    int64_t N;                           // columns per batch
    int64_t mt, nt;                      // work-group tiles along M (128 rows) and N (BN columns)
    int64_t P;                           // tiles computed whole (no K split), tile order
    int KS, spk;                         // the other tiles: K slices of spk stages each
    int64_t X;                           // work-groups numbered by XCD: all (P = 0) or the P whole tiles
    int64_t chunk;                       // X / 8 rounded up
    int64_t nst;                         // stages along K (2 per group)
    GemmBatch bt;
    float * dst;
};

// one stage of staged data in flight (per thread)
struct StageRegs {
    uint4 a[2];                          // activation codes: up to 2 units of 16 B
    uint4 c;                             // weight code chunk (16 B of one row)
    uint4 h;                             // that row's header (Q4_0: .x = the dword with the block's d)
    uint4 s;                             // Q4_K: the column's split sub-block sums
    uint4 q5h;                           // Q5_K: the row's qh chunk (the fifth code bits)
    float x;                             // one activation scale
};

// Q4_K sub-block j's 6-bit scale and min from the 12 scale bytes y|z|w
// (get_scale_min_k4, P01:2164-2176)
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t y, uint32_t z, uint32_t w, uint32_t * sc, uint32_t * mn) {
    const int b8 = 8 * (j & 3);
    if (j < 4) {
        *sc = (y >> b8) & 63;
        *mn = (z >> b8) & 63;
    } else {
        *sc = ((w >> b8) & 0xF) | (((y >> b8) >> 6 & 3) << 4);
        *mn = ((w >> b8) >> 4 & 0xF) | (((z >> b8) >> 6 & 3) << 4);
    }
}

template <int TYPE, int BN>
__global__ __launch_bounds__(kT, 2) void k_gemm2(G2Params p) {   // 2 waves per SIMD: one work-group per CU
    using LY = Lay<TYPE, BN>;
    constexpr bool KQ = LY::KQ;
    constexpr bool Q8 = TYPE == QMM_TYPE_Q8_0;                    // Q4_0's path with plain int8 codes
    constexpr bool IS = LY::IS;                                   // integer sub-block scales (IQ4_XS, Q6_K)
    constexpr bool Q6 = TYPE == QMM_TYPE_Q6_K;
    constexpr bool Q5 = TYPE == QMM_TYPE_Q5_K;                    // Q4_K's path with 5-bit codes
    constexpr bool NLQ = TYPE == QMM_TYPE_IQ4_NL;                 // Q4_0's path through the codebook
    constexpr bool BF = !KQ && !IS;                               // a float scale per block (Q4_0, Q8_0, IQ4_NL)
    constexpr int NWN = BN / 32;                                  // column groups of 32
    constexpr int KSPLIT = 4 / NWN;                               // waves sharing a tile (BN 128: 1, 64: 2)
    constexpr int NQ = 4 / KSPLIT;                                // blocks per stage and wave
    constexpr int NA = BN / 64;                                   // 16-byte code units per thread and stage
    constexpr int kStage = LY::stage;
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // work-group -> tile (mtile-major) and K range.  The first P work-groups take tiles 0 .. P - 1
    // whole, numbered so that those sharing weight rows run on one XCD (work-group b runs on XCD
    // b % 8); the rest take the K slices of tiles P .. in plain order (spread over the XCDs) and add
    // their sums into dst, zeroed from the first such tile's rows by the pre-pass.
    const uint32_t bid = blockIdx.x;                              // grid < 2^31 (host check)
    const uint32_t P = (uint32_t)p.P, X = (uint32_t)p.X, nx = 8 * (uint32_t)p.chunk;
    const uint32_t total = P + (uint32_t)(p.mt * p.nt - p.P) * (uint32_t)p.KS;
    const uint32_t L = bid < nx ? (bid & 7) * (uint32_t)p.chunk + (bid >> 3) : X + (bid - nx);
    if (L >= total || (bid < nx && L >= X)) return;               // uniform
    const uint32_t tile = L < P ? L : P + (L - P) / (uint32_t)p.KS;
    const int ks = L < P ? 0 : (int)((L - P) % (uint32_t)p.KS);
    const bool split = L >= P && p.KS > 1;                        // atomics into zeroed dst
    const uint32_t ntile = tile % (uint32_t)p.nt;
    const int64_t mtile = tile / (uint32_t)p.nt;
    const uint32_t bz = blockIdx.y;
    const int64_t i2 = bz % (uint32_t)p.bt.ne12, i3 = bz / (uint32_t)p.bt.ne12;
    const int64_t mat = i2 / p.bt.r2 + (i3 / p.bt.r3) * p.bt.ne02;
    const int64_t col0 = bz * p.N;                                // first activation column of the batch
    const int64_t n0 = (int64_t)ntile * BN;
    const int s0 = L < P ? 0 : ks * p.spk;
    const int s1 = L < P ? (int)p.nst : (int)((s0 + p.spk) < p.nst ? (s0 + p.spk) : p.nst);   // s1 - s0 is even

    // ---- staging addresses.  Thread tid stages code chunk cs = (tid / 64) % 4 of row tid % 64 of
    // tile tid / 256 (and reads that row's header), NA 16-byte units of activation codes, one
    // activation scale and (Q4_K) one column's sums.  Columns past N are clamped to N - 1: they are
    // computed and never stored.
    const int st_tile = tid >> 8, st_cs = (tid >> 6) & 3, st_row = tid & 63;
    int64_t st_img = 2 * mtile + st_tile;
    st_img = st_img < p.w.ntiles ? st_img : p.w.ntiles - 1;      // a missing second tile re-reads the first
    const uint8_t * tbase = tile_group(p.w, mat, st_img, 0);      // tile-group 0 of the staged tile
    const uint8_t * wbase = tbase + st_row * 16;
    // Q8_0: thread tid stages chunk q8_ch = (tid / 64) % 8 of row tid % 64 of both tiles
    const int q8_ch = (tid >> 6) & 7;
    const uint8_t * wbase8[2];
    if constexpr (Q8) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            int64_t img = 2 * mtile + t;
            img = img < p.w.ntiles ? img : p.w.ntiles - 1;
            wbase8[t] = tile_group(p.w, mat, img, 0) + st_row * 16;
        }
    }
    const int8_t * abase[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) {
        const int u = tid + kT * q;
        const int64_t c = std::min<int64_t>(n0 + (u >> 3), p.N - 1);
        abase[q] = p.xc + (col0 + c) * p.ldk + (u & 7) * 16;
    }
    const int x_blk = BF ? (tid / BN) & 3 : 0;                    // q8_0: 4 blocks x BN columns
    const int64_t x_col = col0 + std::min<int64_t>(n0 + tid % BN, p.N - 1);
    const float * xbase = p.dT + x_col;
    const int8_t * sbase = KQ ? p.bsp + x_col * 16 : nullptr;
    auto fetch = [&](int s) -> StageRegs {
        StageRegs R;
        const int g = s >> 1, hh = s & 1;
#pragma unroll
        for (int q = 0; q < NA; ++q) R.a[q] = *reinterpret_cast<const uint4 *>(abase[q] + s * kSK);
        const uint8_t * tg = wbase + (size_t)g * p.w.tg;
        if constexpr (Q8) {
            // chunks 8 hh .. 8 hh + 7 are blocks 4 hh .. 4 hh + 3 (two halves each); d of the group in chunk 16
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const uint8_t * tgt = wbase8[t] + (size_t)g * p.w.tg;
                const uint4 v = ld16(tgt + (8 * hh + q8_ch) * kChunk);
                const uint32_t dd = *reinterpret_cast<const uint32_t *>(tgt + 16 * kChunk + 8 * hh + 4 * (q8_ch >> 2));
                if (t == 0) { R.c = v; R.h.x = dd; } else { R.s = v; R.h.y = dd; }
            }
        } else {
            R.c = ld16(tg + (4 * hh + st_cs) * kChunk);
        }
        if constexpr (KQ) {
            R.h = ld16(tg + 8 * kChunk);
            R.s = *reinterpret_cast<const uint4 *>(sbase + (int64_t)g * p.ldT * 16);
            if constexpr (Q5) R.q5h = ld16(tg + (9 + (st_cs & 1)) * kChunk);   // qh[16 (cs % 2) ..]
        } else if constexpr (TYPE == QMM_TYPE_IQ4_XS) {
            // the row's 8-byte header {d, scales_h, scales_l[4]} in the tail plane
            const uint2 hd = *reinterpret_cast<const uint2 *>(tbase + (size_t)g * p.w.tg + 8 * kChunk + st_row * 8);
            R.h.x = hd.x;
            R.h.y = hd.y;
        } else if constexpr (Q6) {
            // qh chunk 8 + 2 hh + cs % 2, the stage's 8 scales, d in the tail plane
            R.s = ld16(tg + (8 + 2 * hh + (st_cs & 1)) * kChunk);
            const uint2 sc = *reinterpret_cast<const uint2 *>(tg + 12 * kChunk + 8 * hh);
            R.h.x = sc.x;
            R.h.y = sc.y;
            R.h.z = *reinterpret_cast<const uint16_t *>(tbase + (size_t)g * p.w.tg + 13 * kChunk + st_row * 2);
        } else if constexpr (!Q8) {
            R.h.x = *reinterpret_cast<const uint32_t *>(tg + 8 * kChunk + 4 * (2 * hh + (st_cs >> 1)));
        }
        R.x = xbase[(BF ? (int64_t)s * 4 + x_blk : (int64_t)g) * p.ldT];
        return R;
    };
    auto store = [&](const StageRegs R, int buf, int s) {
        const int hh = s & 1;
        uint8_t * A = lds + buf * kStage;
        uint8_t * B = A + LY::oB;
        uint8_t * W = A + LY::oW;
        float * X = reinterpret_cast<float *>(A + LY::oX);
#pragma unroll
        for (int q = 0; q < NA; ++q) {
            const int u = tid + kT * q;
            *reinterpret_cast<uint4 *>(A + (u >> 3) * kAP + (u & 7) * 16) = R.a[q];
        }
        const uint32_t e[4] = { R.c.x, R.c.y, R.c.z, R.c.w };
        if constexpr (Q8) {
            // chunk ch of the stage = half ch % 2 of block ch / 2: the layout of the B planes as is
            *reinterpret_cast<uint4 *>(B + q8_ch * kChunk + st_row * 16) = R.c;
            *reinterpret_cast<uint4 *>(B + (8 + q8_ch) * kChunk + st_row * 16) = R.s;
            if ((q8_ch & 1) == 0) {                               // d of block ch / 2 of the stage
                const int blk = q8_ch >> 1;
                float * wd = reinterpret_cast<float *>(W) + blk * 64 + st_row;
                wd[0] = h2f(R.h.x >> (16 * (blk & 1)));
                wd[4 * 64] = h2f(R.h.y >> (16 * (blk & 1)));
            }
            if (tid < 4 * BN) X[tid] = R.x;                       // [block][col]
        } else if constexpr (TYPE == QMM_TYPE_IQ4_XS) {
            // chunk 4 hh + cs is sub-block cs of the stage: low nibbles k < 16, high nibbles k >= 16,
            // through the codebook; its scale ls - 32 (P01:3390-3398)
            uint4 lo, hi;
            lo.x = iq4_lookup(e[0] & 0x0F0F0F0Fu); hi.x = iq4_lookup((e[0] >> 4) & 0x0F0F0F0Fu);
            lo.y = iq4_lookup(e[1] & 0x0F0F0F0Fu); hi.y = iq4_lookup((e[1] >> 4) & 0x0F0F0F0Fu);
            lo.z = iq4_lookup(e[2] & 0x0F0F0F0Fu); hi.z = iq4_lookup((e[2] >> 4) & 0x0F0F0F0Fu);
            lo.w = iq4_lookup(e[3] & 0x0F0F0F0Fu); hi.w = iq4_lookup((e[3] >> 4) & 0x0F0F0F0Fu);
            uint8_t * b = B + ((st_tile * 4 + st_cs) * 2) * kChunk + st_row * 16;
            *reinterpret_cast<uint4 *>(b) = lo;
            *reinterpret_cast<uint4 *>(b + kChunk) = hi;
            const int ib = 4 * hh + st_cs;
            const int ls = (int)(((R.h.y >> (4 * ib)) & 0xFu) | ((((R.h.x >> 16) >> (2 * ib)) & 3u) << 4));
            reinterpret_cast<int *>(W)[((st_tile * 4 + st_cs) * 2) * 64 + st_row] = ls - 32;
            if (st_cs == 0) reinterpret_cast<float *>(W + 2 * 4 * 2 * 64 * 4)[st_tile * 64 + st_row] = h2f(R.h.x);
            if (tid < BN) X[tid] = R.x;
        } else if constexpr (Q6) {
            // ql chunk 4 hh + cs: low nibbles of block cs / 2, high nibbles of block cs / 2 + 2, both half
            // lh = cs % 2 (16 weights); qh bits 2 g .. 2 g + 1 of chunk 8 + 2 hh + lh; code - 32
            const int lh = st_cs & 1, gl = st_cs >> 1;
            const uint32_t qh[4] = { R.s.x, R.s.y, R.s.z, R.s.w };
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int g = gl + 2 * t;
                uint32_t v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t c = ((e[i] >> (4 * t)) & 0x0F0F0F0Fu) | (((qh[i] >> (2 * g)) & 0x03030303u) << 4);
                    v[i] = ((c | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
                }
                *reinterpret_cast<uint4 *>(B + ((st_tile * 4 + g) * 2 + lh) * kChunk + st_row * 16) =
                    make_uint4(v[0], v[1], v[2], v[3]);
                const uint32_t scw = t ? R.h.y : R.h.x;           // scales 8 hh + 4 t .. + 3
                reinterpret_cast<int *>(W)[((st_tile * 4 + g) * 2 + lh) * 64 + st_row] =
                    (int)(int8_t)((scw >> (8 * st_cs)) & 0xffu);
            }
            if (st_cs == 0) reinterpret_cast<float *>(W + 2 * 4 * 2 * 64 * 4)[st_tile * 64 + st_row] = h2f(R.h.z);
            if (tid < BN) X[tid] = R.x;
        } else if constexpr (!KQ) {
            // chunk 4 hh + cs is block cs of the stage: low nibbles k < 16, high nibbles k >= 16
            // (IQ4_NL: the codebook value)
            auto dec = [](uint32_t nib) { return NLQ ? iq4_lookup(nib) : q4_minus8(nib); };
            uint4 lo, hi;
            lo.x = dec(e[0] & 0x0F0F0F0Fu); hi.x = dec((e[0] >> 4) & 0x0F0F0F0Fu);
            lo.y = dec(e[1] & 0x0F0F0F0Fu); hi.y = dec((e[1] >> 4) & 0x0F0F0F0Fu);
            lo.z = dec(e[2] & 0x0F0F0F0Fu); hi.z = dec((e[2] >> 4) & 0x0F0F0F0Fu);
            lo.w = dec(e[3] & 0x0F0F0F0Fu); hi.w = dec((e[3] >> 4) & 0x0F0F0F0Fu);
            uint8_t * b = B + ((st_tile * 4 + st_cs) * 2) * kChunk + st_row * 16;
            *reinterpret_cast<uint4 *>(b) = lo;
            *reinterpret_cast<uint4 *>(b + kChunk) = hi;
            // d of block cs of the stage (block 4 hh + cs of the group)
            reinterpret_cast<float *>(W)[(st_tile * 4 + st_cs) * 64 + st_row] = h2f(R.h.x >> (16 * (st_cs & 1)));
            if (tid < 4 * BN) X[tid] = R.x;                       // [block][col]
        } else {
            // chunk 4 hh + cs holds weights 16 h .. 16 h + 15 (h = cs % 2) of sub-blocks 4 hh + ql (low
            // nibbles) and 4 hh + ql + 1 (high nibbles), ql = 2 (cs / 2)
            const int h = st_cs & 1, ql = 2 * (st_cs >> 1);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                uint32_t sc, mn;
                q4k_scale_min((4 * hh + ql + t) ^ (QMM_RED == 5), R.h.y, R.h.z, R.h.w, &sc, &mn);   // (mutation 5)
                const uint32_t sh = sc >> 3, sl = sc & 7;
                uint4 vh, vl;
                const uint32_t m0 = (e[0] >> (4 * t)) & 0x0F0F0F0Fu, m1 = (e[1] >> (4 * t)) & 0x0F0F0F0Fu;
                const uint32_t m2 = (e[2] >> (4 * t)) & 0x0F0F0F0Fu, m3 = (e[3] >> (4 * t)) & 0x0F0F0F0Fu;
                vh.x = v2_mul(m0, sh); vl.x = v2_mul(m0, sl);
                vh.y = v2_mul(m1, sh); vl.y = v2_mul(m1, sl);
                vh.z = v2_mul(m2, sh); vl.z = v2_mul(m2, sl);
                vh.w = v2_mul(m3, sh); vl.w = v2_mul(m3, sl);
                if constexpr (Q5) {
                    // (q - 16) s = q4 s - 16 s (1 - hb), hb = bit j of qh (j = the sub-block): q4 s < 128, so
                    // the offset-binary subtract borrows nothing across bytes; the result is in [-112, 105]
                    const int j = 4 * hh + ql + t;
                    auto fix = [&](uint32_t v, uint32_t qh, uint32_t s) {
                        const uint32_t nhb = (~qh >> j) & 0x01010101u;
                        return ((v | 0x80808080u) - v2_mul(nhb, 16 * s)) ^ 0x80808080u;
                    };
                    vh.x = fix(vh.x, R.q5h.x, sh); vl.x = fix(vl.x, R.q5h.x, sl);
                    vh.y = fix(vh.y, R.q5h.y, sh); vl.y = fix(vl.y, R.q5h.y, sl);
                    vh.z = fix(vh.z, R.q5h.z, sh); vl.z = fix(vl.z, R.q5h.z, sl);
                    vh.w = fix(vh.w, R.q5h.w, sh); vl.w = fix(vl.w, R.q5h.w, sl);
                }
                uint8_t * b = B + (((st_tile * 4 + ql + t) * 2 + h) * 2) * kChunk + st_row * 16;
                *reinterpret_cast<uint4 *>(b) = vh;
                *reinterpret_cast<uint4 *>(b + kChunk) = vl;
            }
            {                                                     // mins 2 cs and 2 cs + 1 of the row (4 B: 2 mins, 2 zeros)
                uint32_t sc, m0, m1;
                q4k_scale_min(2 * st_cs, R.h.y, R.h.z, R.h.w, &sc, &m0);
                q4k_scale_min(2 * st_cs + 1, R.h.y, R.h.z, R.h.w, &sc, &m1);
                uint16_t * mw = reinterpret_cast<uint16_t *>(W + (st_tile * 64 + st_row) * 16);
                mw[st_cs] = (uint16_t)(m0 | (m1 << 8));
                if constexpr (Q5) {                               // scales 2 cs, 2 cs + 1 after the mins
                    uint32_t s0, s1, mm;
                    q4k_scale_min(2 * st_cs, R.h.y, R.h.z, R.h.w, &s0, &mm);
                    q4k_scale_min(2 * st_cs + 1, R.h.y, R.h.z, R.h.w, &s1, &mm);
                    mw[4 + st_cs] = (uint16_t)(s0 | (s1 << 8));
                } else {
                    mw[4 + st_cs] = 0;
                }
            }
            if (st_cs == 0)                                       // d and dmin
                reinterpret_cast<float2 *>(W + 2 * 64 * 16)[st_tile * 64 + st_row] = make_float2(h2f(R.h.x), h2f(R.h.x >> 16));
            if (tid < BN) {
                X[tid] = R.x;
                *reinterpret_cast<uint4 *>(A + LY::oS + tid * 16) = R.s;
            }
        }
    };

    // ---- per-wave tile: image tile wr (64 rows = 2 MFMA row tiles) x columns wn * 32 .. + 32,
    // blocks wk, wk + KSPLIT, ... of every stage
    const int wr = wave & 1, wn = (wave >> 1) % NWN, wk = (wave >> 1) / NWN;
    const int h = lane >> 5, l32 = lane & 31;
    v16f out0 = v16f{}, out1 = v16f{};                            // row tiles 0 and 1
    v16i c1[2], c2[2];                                            // Q4_K: set by each super-block's first MFMAs
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        c1[rt] = v16i{};
        c2[rt] = v16i{};
    }
    v16i magic;
#pragma unroll
    for (int r = 0; r < 16; ++r) magic[r] = kMagic;

    // operands of one block (Q4_0) / sub-block (Q4_K); Q4_0 loads them from LDS one block ahead of
    // the MFMAs that use them (two register sets)
    struct Ops {
        v4i a;                           // activation codes of this wave's 32 columns
        v4i b[2][2];                     // [row tile][0: q - 8 (Q4_0) or q * sh (Q4_K), 1: q * sl]
        float dw[2];                     // Q4_0, Q8_0: d_w of the lane's rows
        float dx[16];                    // Q4_0, Q8_0: d_x of the lane's 16 columns
        int sc[2][2];                    // IQ4_XS, Q6_K: [row tile][16-weight half] integer scale
    };
    auto load_ops = [&](int buf, int q) -> Ops {
        Ops o;
        const uint8_t * A = lds + buf * kStage + (wn * 32 + l32) * kAP + 16 * h;
        const uint8_t * B = lds + buf * kStage + LY::oB;
        const uint8_t * W = lds + buf * kStage + LY::oW;
        const float * X = reinterpret_cast<const float *>(lds + buf * kStage + LY::oX);
        o.a = *reinterpret_cast<const v4i *>(A + q * 32);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int row = 32 * rt + l32;
            if constexpr (BF) {
                o.b[rt][0] = *reinterpret_cast<const v4i *>(B + ((wr * 4 + q) * 2 + h) * kChunk + row * 16);
                o.dw[rt] = reinterpret_cast<const float *>(W)[(wr * 4 + q) * 64 + row];
            } else if constexpr (IS) {
                o.b[rt][0] = *reinterpret_cast<const v4i *>(B + ((wr * 4 + q) * 2 + h) * kChunk + row * 16);
                o.sc[rt][0] = reinterpret_cast<const int *>(W)[((wr * 4 + q) * 2) * 64 + row];
                if constexpr (Q6) o.sc[rt][1] = reinterpret_cast<const int *>(W)[((wr * 4 + q) * 2 + 1) * 64 + row];
            } else {
                const uint8_t * b = B + (((wr * 4 + q) * 2 + h) * 2) * kChunk + row * 16;
                o.b[rt][0] = *reinterpret_cast<const v4i *>(b);
                o.b[rt][1] = *reinterpret_cast<const v4i *>(b + kChunk);
            }
        }
        if constexpr (BF) {
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const float4 v = *reinterpret_cast<const float4 *>(X + q * BN + wn * 32 + 8 * g4 + 4 * h);
                o.dx[4 * g4] = v.x; o.dx[4 * g4 + 1] = v.y; o.dx[4 * g4 + 2] = v.z; o.dx[4 * g4 + 3] = v.w;
            }
        }
        return o;
    };
    // first: the super-block's first (sub-)block of this wave (Q4_K): its MFMAs start from an
    // inline zero instead of cleared accumulators
    auto mma = [&](const Ops o, bool first) {
        if constexpr (BF) {
            const v16i d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, o.b[0][0], magic, 0, 0, 0);
            const v16i d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, o.b[1][0], magic, 0, 0, 0);
            const float nm0 = -12582912.0f * o.dw[0], nm1 = -12582912.0f * o.dw[1];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int di = d0[r];                             // (bit_cast of a vector element reads element 0)
                out0[r] = __builtin_fmaf(__builtin_fmaf(__builtin_bit_cast(float, di), o.dw[0], nm0), o.dx[r], out0[r]);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int di = d1[r];
                out1[r] = __builtin_fmaf(__builtin_fmaf(__builtin_bit_cast(float, di), o.dw[1], nm1), o.dx[r], out1[r]);
            }
            // keep this block's products from being deferred past later MFMAs (register pressure)
            asm volatile("" : "+v"(out0), "+v"(out1));
        } else if constexpr (IS) {
            // the (sub-)block dot from a fresh MFMA, times its integer scale into isum (c1).  Q6_K's
            // scale changes every 16 weights: one MFMA per lane half, the other half's operand zero.
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                if constexpr (!Q6) {
                    const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, o.b[rt][0], v16i{}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) c1[rt][r] += o.sc[rt][0] * d[r];
                } else {
                    const v4i zero = v4i{ 0, 0, 0, 0 };
                    const v16i d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, h ? zero : o.b[rt][0], v16i{}, 0, 0, 0);
                    const v16i d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, h ? o.b[rt][0] : zero, v16i{}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) c1[rt][r] += o.sc[rt][0] * d0[r] + o.sc[rt][1] * d1[r];
                }
            }
        } else if (first) {
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                c1[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, o.b[rt][0], v16i{}, 0, 0, 0);
                c2[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, o.b[rt][1], v16i{}, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                c1[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, o.b[rt][0], c1[rt], 0, 0, 0);
                c2[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, o.b[rt][1], c2[rt], 0, 0, 0);
            }
        }
    };
    auto compute = [&](int buf, int s) {
        if constexpr (BF) {
            Ops o0 = load_ops(buf, wk), o1;
#pragma unroll
            for (int i = 0; i < NQ; ++i) {
                if (i + 1 < NQ) o1 = load_ops(buf, wk + (i + 1) * KSPLIT);
                __builtin_amdgcn_sched_barrier(0);
                mma(o0, false);
                __builtin_amdgcn_sched_barrier(0);
                o0 = o1;
            }
        } else if (KQ && (s & 1) == 0) {                          // uniform: a super-block starts
            mma(load_ops(buf, wk), true);
#pragma unroll
            for (int i = 1; i < NQ; ++i) mma(load_ops(buf, wk + i * KSPLIT), false);
        } else {                                                  // (registers: no second operand set)
#pragma unroll
            for (int i = 0; i < NQ; ++i) mma(load_ops(buf, wk + i * KSPLIT), false);
        }
        if constexpr (IS) {
            if (s & 1) {                                          // end of the super-block (uniform)
                const float * X = reinterpret_cast<const float *>(lds + buf * kStage + LY::oX);
                const float * Wd = reinterpret_cast<const float *>(lds + buf * kStage + LY::oW + 2 * 4 * 2 * 64 * 4);
                float dx[16];
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const float4 v = *reinterpret_cast<const float4 *>(X + wn * 32 + 8 * g4 + 4 * h);
                    dx[4 * g4] = v.x; dx[4 * g4 + 1] = v.y; dx[4 * g4 + 2] = v.z; dx[4 * g4 + 3] = v.w;
                }
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const float d = Wd[wr * 64 + 32 * rt + l32];
                    v16f & o = rt ? out1 : out0;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int is = c1[rt][r];
                        o[r] = __builtin_fmaf(dx[r], d * (float)is, o[r]);
                    }
                    c1[rt] = v16i{};
                }
            }
        }
        if constexpr (KQ) {
            if (s & 1) {                                          // end of the super-block (uniform)
                const uint8_t * W = lds + buf * kStage + LY::oW;
                const float * X = reinterpret_cast<const float *>(lds + buf * kStage + LY::oX);
                const v4i sv = *reinterpret_cast<const v4i *>(lds + buf * kStage + LY::oS + (wn * 32 + l32) * 16);
                float dx[16];
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const float4 v = *reinterpret_cast<const float4 *>(X + wn * 32 + 8 * g4 + 4 * h);
                    dx[4 * g4] = v.x; dx[4 * g4 + 1] = v.y; dx[4 * g4 + 2] = v.z; dx[4 * g4 + 3] = v.w;
                }
                // min term (one wave of the tile): k in [0, 8) of lane half 0 carries sub-blocks 0..7
                const v4i zero = v4i{ 0, 0, 0, 0 };
                const v4i ah = h ? zero : v4i{ sv.x, sv.y, 0, 0 };
                const v4i al = h ? zero : v4i{ sv.z, sv.w, 0, 0 };
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const int row = wr * 64 + 32 * rt + l32;
                    const float2 dd = reinterpret_cast<const float2 *>(W + 2 * 64 * 16)[row];
                    const v4i bmin = h ? zero : *reinterpret_cast<const v4i *>(W + row * 16);
                    // (KSPLIT 2: the tile's second wave adds no min term; its sums meet wave 0's)
                    v16i mh = v16i{}, ml = v16i{};
                    if (KSPLIT == 1 || wk == 0) {
                        if constexpr (Q5) {
                            // sum_j sc_j bsum_j (k 8..15 of the row) times 16, into c2 (isc = 8 c1 + c2) one
                            // MFMA result at a time
                            const v4i ash = h ? zero : v4i{ 0, 0, sv.x, sv.y };
                            const v4i asl = h ? zero : v4i{ 0, 0, sv.z, sv.w };
                            const v16i sh = __builtin_amdgcn_mfma_i32_32x32x32_i8(ash, bmin, v16i{}, 0, 0, 0);
#pragma unroll
                            for (int r = 0; r < 16; ++r) c2[rt][r] += 1024 * sh[r];
                            __builtin_amdgcn_sched_barrier(0);
                            const v16i sl = __builtin_amdgcn_mfma_i32_32x32x32_i8(asl, bmin, v16i{}, 0, 0, 0);
#pragma unroll
                            for (int r = 0; r < 16; ++r) c2[rt][r] += 16 * sl[r];
                            __builtin_amdgcn_sched_barrier(0);
                        }
                        mh = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, bmin, v16i{}, 0, 0, 0);
                        ml = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, bmin, v16i{}, 0, 0, 0);
                    }
                    v16f & o = rt ? out1 : out0;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int isc = 8 * c1[rt][r] + c2[rt][r];
                        const int imn = 64 * mh[r] + ml[r];
                        o[r] += dx[r] * (dd.x * (float)isc - dd.y * (float)imn);
                    }
                }
            }
        }
    };

    // ---- K loop.  Q4_0: stages in pairs; the data of a stage is fetched two stages before it is
    // computed (two register sets) and stored to LDS during the stage before it (two LDS buffers).  Inside a
    // stage, computing it and storing the next touch different buffers, so the order is free: waves
    // 0-3 compute first and waves 4-7 (the second wave on each SIMD) store first, which keeps one wave
    // per SIMD on the MFMAs while the other unpacks weights.  Fetches past the slice re-read its last
    // stage (unconditional loads keep the wait counts static).
    const bool store_first = wave >= 4;
    if constexpr (!KQ) {
        StageRegs R0 = fetch(s0), R1 = fetch(s0 + 1);
        store(R0, 0, s0);
        __syncthreads();
        for (int s = s0; s < s1; s += 2) {                        // uniform over the work-group
            R0 = fetch(std::min(s + 2, s1 - 1));
            if (store_first) store(R1, 1, s + 1);
            compute(0, s);
            if (!store_first) store(R1, 1, s + 1);
            __syncthreads();
            R1 = fetch(std::min(s + 3, s1 - 1));
            if (store_first && s + 2 < s1) store(R0, 0, s + 2);
            compute(1, s + 1);
            if (!store_first && s + 2 < s1) store(R0, 0, s + 2);
            __syncthreads();
        }
    } else {                                                      // Q4_K (registers): one stage ahead
        StageRegs R = fetch(s0);
        store(R, 0, s0);
        __syncthreads();
        for (int s = s0; s < s1; ++s) {
            R = fetch(std::min(s + 1, s1 - 1));
            compute((s - s0) & 1, s);
            if (s + 1 < s1) store(R, (s - s0 + 1) & 1, s + 1);
            __syncthreads();
        }
    }

    // ---- the two waves of a tile (BN = 64) add their sums through LDS
    if constexpr (KSPLIT == 2) {
        float * red = reinterpret_cast<float *>(lds) + ((wr + 2 * wn) * 32) * 64 + lane;
        if (wk == 1) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                red[r * 64] = out0[r];
                red[(16 + r) * 64] = out1[r];
            }
        }
        __syncthreads();
        if (wk == 1) return;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            out0[r] += red[r * 64];
            out1[r] += red[(16 + r) * 64];
        }
    }

    // ---- store: lane holds row 32 rt + l32 of its image tile for 16 columns
    float * dst = p.dst + i2 * p.bt.d_nb2 + i3 * p.bt.d_nb3;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const int64_t m = (2 * mtile + wr) * kTileRows + 32 * rt + l32;
        if (m >= p.w.M) continue;
        const v16f v = rt ? out1 : out0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t n = n0 + wn * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (n < p.N) {
                float * o = dst + n * p.bt.d_nb1 + m;
                const float x = v[r];
                if (!split) *o = x;
                else atomicAdd(o, x);
            }
        }
    }
}

template <int TYPE, int BN>
hipError_t launch_t(const G2Params & p, const dim3 & g, hipStream_t s, const KTime * kt) {
    constexpr int lds = 2 * Lay<TYPE, BN>::stage;
    static const hipError_t attr =
        hipFuncSetAttribute((const void *)k_gemm2<TYPE, BN>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return attr;
    if (kt) hipExtLaunchKernelGGL(k_gemm2<TYPE, BN>, g, dim3(kT), (uint32_t)lds, s, kt->start, kt->stop, 0, p);
    else k_gemm2<TYPE, BN><<<g, kT, lds, s>>>(p);
    return hipGetLastError();
}

// Launch shape: column tile BN, and which tiles split K how, from a cost
// model fitted to measurements on MI355X: a work-group stage costs ~2 us at
// BN = 128 and 0.62 of that at BN = 64 (the weight staging and the barrier do
// not shrink with the tile); work-groups run in rounds of one per CU; K
// slices add their partial sums with float atomics (~480 adds per ns over the
// chip), into dst rows the pre-pass zeroed.  Two kinds of candidate, each
// priced as rounds x stages x stage cost + atomics, the cheapest taken:
//  * uniform: every tile in KS slices of spk stages;
//  * tail (one batch): the tiles of the whole rounds (P, in whole rows of
//    column tiles) unsplit, the rest in KS slices that fill the last round.
struct G2Shape {
    int BN, KS, spk;
    int64_t mt, nt, P;
};
// (Q5_K takes 64-column tiles only: at 128 its registers spill)
G2Shape g2_shape(int type, const WView & w, int64_t N, int64_t nbatch) {
    static const int64_t cus = [] {
        const char * e = getenv("QMM_GEMM_CUS");
        return e ? std::max<int64_t>(1, atoll(e)) : (int64_t)256;
    }();
    const char * te = getenv("QMM_GEMM_TAIL");
    const bool tail_on = !te || atoi(te) != 0;
    G2Shape best{};
    double best_us = 1e300;
    const int64_t mt = (w.M + 127) / 128, nst = 2 * w.G;
    auto consider = [&](double us, const G2Shape & sh) {
        if (us < best_us * 0.98) {                                // prefer the earlier (wider, unsplit) shape on ties
            best_us = us;
            best = sh;
        }
    };
    for (int bn : { 128, 64 }) {
        if (bn == 128 && type == QMM_TYPE_Q5_K) continue;
        const double c = 2.0 * (bn == 64 ? 0.62 : 1.0);           // us per stage
        const int64_t nt = (N + bn - 1) / bn, T = mt * nt;
        int64_t prev_gps = -1;
        for (int64_t ks = 1; ks <= std::min<int64_t>(w.G, 64); ++ks) {
            const int64_t gps = (w.G + ks - 1) / ks;
            if (gps == prev_gps) continue;                        // same split as a smaller ks
            prev_gps = gps;
            const int64_t kss = (w.G + gps - 1) / gps;
            const int64_t wgs = T * nbatch * kss;
            double us = (double)((wgs + cus - 1) / cus) * (double)(2 * gps) * c;
            if (kss > 1) us += (double)w.M * (double)N * (double)nbatch * (double)kss / 480000.0;
            consider(us, G2Shape{ bn, (int)kss, (int)(2 * gps), mt, nt, 0 });
        }
        if (!tail_on || nbatch != 1 || T <= cus) continue;
        const int64_t R = T / cus, P = (R * cus / nt) * nt, tail = T - P;
        if (P <= 0 || tail <= 0) continue;
        prev_gps = -1;
        for (int64_t ks = 2; ks <= std::min<int64_t>(w.G, 64); ++ks) {
            const int64_t gps = (w.G + ks - 1) / ks;
            if (gps == prev_gps) continue;
            prev_gps = gps;
            const int64_t kss = (w.G + gps - 1) / gps;
            // slices first fill the slots the whole rounds leave free, then rounds of their own
            const int64_t free_slots = (R * cus - P) * std::max<int64_t>(1, nst / (2 * gps));
            const int64_t rest = std::max<int64_t>(0, tail * kss - free_slots);
            double us = (double)R * (double)nst * c + (double)((rest + cus - 1) / cus) * (double)(2 * gps) * c;
            us += (double)tail * (double)bn * 128.0 * (double)kss / 480000.0;
            consider(us, G2Shape{ bn, (int)kss, (int)(2 * gps), mt, nt, P });
        }
    }
    return best;
}

}  // namespace

int gemm_kslices(int type, const WView & w, int64_t N, int64_t nbatch) { return g2_shape(type, w, N, nbatch).KS; }

int64_t gemm_zero_from(int type, const WView & w, int64_t N, int64_t nbatch) {
    const G2Shape sh = g2_shape(type, w, N, nbatch);
    if (sh.KS == 1) return w.M;                                   // nothing adds into dst
    return std::min<int64_t>(w.M, sh.P / sh.nt * 128);
}

void gemm_shape(int type, const WView & w, int64_t N, int64_t nbatch, int64_t * workgroups, int * threads,
                int * lds_bytes) {
    const G2Shape sh = g2_shape(type, w, N, nbatch);
    *workgroups = (sh.P + (sh.mt * sh.nt - sh.P) * sh.KS) * nbatch;
    *threads = kT;
    int st;
    switch (type) {
        case QMM_TYPE_Q4_K:
        case QMM_TYPE_Q5_K: st = sh.BN == 64 ? Lay<QMM_TYPE_Q4_K, 64>::stage : Lay<QMM_TYPE_Q4_K, 128>::stage; break;
        case QMM_TYPE_Q6_K:
        case QMM_TYPE_IQ4_XS: st = sh.BN == 64 ? Lay<QMM_TYPE_Q6_K, 64>::stage : Lay<QMM_TYPE_Q6_K, 128>::stage; break;
        default: st = sh.BN == 64 ? Lay<QMM_TYPE_Q4_0, 64>::stage : Lay<QMM_TYPE_Q4_0, 128>::stage; break;
    }
    *lds_bytes = 2 * st;
}

hipError_t launch_gemm(int type, const WView & w, const ActBuf & a, int64_t N, int64_t nbatch, const GemmBatch & bt,
                       float * dst, hipStream_t s, const KTime * kt) {
    if (!a.dT || a.ldk != w.G * 256 || a.ldT < N * nbatch + 64 || N <= 0 || nbatch <= 0 ||
        nbatch > 65535 || a.vdt != vec_dot_type(type) || ((type == QMM_TYPE_Q4_K || type == QMM_TYPE_Q5_K) && !a.bsp))
        return hipErrorInvalidValue;
    const G2Shape sh = g2_shape(type, w, N, nbatch);
    G2Params p{};
    p.w = w;
    p.xc = a.codes;
    p.ldk = a.ldk;
    p.dT = a.dT;
    p.ldT = a.ldT;
    p.bsp = a.bsp;
    p.N = N;
    p.mt = sh.mt;
    p.nt = sh.nt;
    p.nst = 2 * w.G;
    p.KS = sh.KS;
    p.spk = sh.spk;
    p.P = sh.P;
    p.bt = bt;
    p.dst = dst;
    const int64_t total = sh.P + (p.mt * p.nt - sh.P) * p.KS;
    p.X = sh.P > 0 ? sh.P : total;
    p.chunk = (p.X + 7) / 8;
    const int64_t grid = 8 * p.chunk + (total - p.X);
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 g((unsigned)grid, (unsigned)nbatch);
    if (type == QMM_TYPE_Q4_0)
        return sh.BN == 64 ? launch_t<QMM_TYPE_Q4_0, 64>(p, g, s, kt) : launch_t<QMM_TYPE_Q4_0, 128>(p, g, s, kt);
    if (type == QMM_TYPE_Q8_0)
        return sh.BN == 64 ? launch_t<QMM_TYPE_Q8_0, 64>(p, g, s, kt) : launch_t<QMM_TYPE_Q8_0, 128>(p, g, s, kt);
    if (type == QMM_TYPE_Q6_K)
        return sh.BN == 64 ? launch_t<QMM_TYPE_Q6_K, 64>(p, g, s, kt) : launch_t<QMM_TYPE_Q6_K, 128>(p, g, s, kt);
    if (type == QMM_TYPE_IQ4_XS)
        return sh.BN == 64 ? launch_t<QMM_TYPE_IQ4_XS, 64>(p, g, s, kt) : launch_t<QMM_TYPE_IQ4_XS, 128>(p, g, s, kt);
    if (type == QMM_TYPE_Q4_K)
        return sh.BN == 64 ? launch_t<QMM_TYPE_Q4_K, 64>(p, g, s, kt) : launch_t<QMM_TYPE_Q4_K, 128>(p, g, s, kt);
    if (type == QMM_TYPE_Q5_K)
        return launch_t<QMM_TYPE_Q5_K, 64>(p, g, s, kt);         // g2_shape takes BN = 64 only
    if (type == QMM_TYPE_IQ4_NL)
        return sh.BN == 64 ? launch_t<QMM_TYPE_IQ4_NL, 64>(p, g, s, kt) : launch_t<QMM_TYPE_IQ4_NL, 128>(p, g, s, kt);
    return hipErrorInvalidValue;
}

}  // namespace qmm
