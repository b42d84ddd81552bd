// k_gemm2.hip - prefill GEMM (N >= 16 columns) for Q4_0 and Q4_K on gfx950
// v_mfma_i32_32x32x32_i8.
//
// Role of the reference's int8 prefill GEMMs (kernel_mul_mm_kq2d_q4_0_i8,
// P0099:377-455, and kernel_mul_mm_kq2d_q4_K_i8, P01:1919-2024), redesigned
// for CDNA4 and for ggml-cpu's numerics:
//  * a work-group owns 128 weight rows (two 64-row tiles of the weight image)
//    x 128 activation columns and walks K in stages of 128 (half a group);
//    per stage it stages in LDS the activation codes of its columns (a padded
//    pitch spreads the rows over the banks), the stage's chunk planes of its
//    two tiles (as laid out in HBM: the 16 bytes of a row are one MFMA
//    operand) and the activation scales, double-buffered one stage ahead;
//  * each of the 4 waves computes 64 rows x 64 columns as 2 x 2 MFMA tiles
//    of 32 x 32, one 32-weight (sub-)block per MFMA.  Both operands place
//    k in [16h, 16h + 16) of the block in lane half h, so the int32 result is
//    the block's exact integer dot, as in ggml_vec_dot_*;
//  * Q4_0: the weight operand is q - 8 (bytewise), and the float combine of
//    every block, acc += (float)dot * (d_w * d_x), runs on the VALU as in
//    ggml's vec_dot_q4_0_q8_0;
//  * Q4_K: the 6-bit sub-block scale sc = 8 sh + sl is folded into two int8
//    operands q * sh and q * sl (a packed 16-bit multiply scales 4 codes at
//    once; every product is < 128), and the min term is a third MFMA against
//    the sub-block's min replicated (m * sum of the block's codes), so the
//    whole super-block accumulates inside the MFMA in int32 and the float
//    combine runs once per 256 weights;
//  * work-groups are numbered so that those sharing weight rows land on the
//    same XCD; short matrices split K over KS work-groups that add their
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
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

constexpr int kT = 512;                  // threads per work-group (8 waves)
constexpr int kBN = 128;                 // activation columns per work-group
constexpr int kSK = 128;                 // k per stage
constexpr int kAP = kSK + 16;            // LDS pitch of one column's codes
constexpr int kAB = kBN * kAP;           // A stage bytes
constexpr int kBB = 2 * 5 * kChunk;      // B stage bytes: 2 tiles x (4 code chunks + header)
constexpr int kXB = 4 * kBN * 4;         // scale stage bytes (4 blocks x 128 columns, f32)
constexpr int kStage = kAB + kBB + kXB;  // 30720

struct G2Params {
    WView w;
    const int8_t * xc;                   // activation codes [col][ldk]
    int64_t ldk;
    const float * dT;                    // activation scales [block][ldT]
    int64_t ldT;
    int64_t N;                           // columns per batch
    int64_t mt, nt;                      // work-group tiles along M (128 rows) and N (128 columns)
    int64_t chunk;                       // work-groups per XCD (numbering)
    int KS, spk;                         // K slices, stages per slice
    int64_t nst;                         // stages along K (2 per group)
    GemmBatch bt;
    float * dst;
};

__device__ __forceinline__ uint32_t v2_mul(uint32_t v, uint32_t s) {   // 4 bytes x s, no carries (products < 256)
    const v2u16 a = __builtin_bit_cast(v2u16, v);
    const v2u16 b = { (unsigned short)s, (unsigned short)s };
    return __builtin_bit_cast(uint32_t, a * b);
}

template <int TYPE>
__global__ __launch_bounds__(kT) void k_gemm2(G2Params p) {
    constexpr bool KQ = TYPE == QMM_TYPE_Q4_K;
    constexpr int UQ = KQ ? 4 : 1;                                // Q4_0: one block's products live at a time
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t bid = blockIdx.x;
    const int64_t L = (bid & 7) * p.chunk + (bid >> 3);
    if (L >= p.mt * p.nt * p.KS) return;                          // uniform
    const int64_t ntile = L % p.nt, rest = L / p.nt;
    const int ks = (int)(rest % p.KS);
    const int64_t mtile = rest / p.KS;
    const int64_t bz = blockIdx.y;
    const int64_t i2 = bz % p.bt.ne12, i3 = bz / p.bt.ne12;
    const int64_t mat = i2 / p.bt.r2 + (i3 / p.bt.r3) * p.bt.ne02;
    const int64_t col0 = bz * p.N;                                // first activation column of the batch
    const int64_t n0 = ntile * kBN;
    const int s0 = ks * p.spk;
    const int s1 = (int)((s0 + p.spk) < p.nst ? (s0 + p.spk) : p.nst);

    // ---- staging of one stage: global -> registers (fetch), registers -> LDS (store)
    constexpr int kNA = kBN * kSK / 16 / kT;                      // 16-byte code units per thread
    constexpr int kNB = (kBB / 16 + kT - 1) / kT;                 // 16-byte weight units per thread
    uint4 ra[kNA], rb[kNB];
    float4 rx;
    auto fetch = [&](int s) {
        const int64_t g = s >> 1, hh = s & 1;
#pragma unroll
        for (int q = 0; q < kNA; ++q) {                           // codes: 128 columns x 8 units
            const int u = tid + kT * q, c = u >> 3, un = u & 7;
            ra[q] = make_uint4(0, 0, 0, 0);
            if (n0 + c < p.N) ra[q] = *reinterpret_cast<const uint4 *>(p.xc + (col0 + n0 + c) * p.ldk + s * kSK + un * 16);
        }
#pragma unroll
        for (int q = 0; q < kNB; ++q) {                           // weights: 2 tiles x 5 chunks x 64 rows
            const int u = tid + kT * q;
            rb[q] = make_uint4(0, 0, 0, 0);
            if (u < kBB / 16) {
                const int tt = u / 320, rem = u - tt * 320, cs = rem >> 6, r = rem & 63;
                int64_t tile = 2 * mtile + tt;
                tile = tile < p.w.ntiles ? tile : p.w.ntiles - 1;
                const int c = cs < 4 ? 4 * (int)hh + cs : 8;
                rb[q] = ld16_nt(tile_group(p.w, mat, tile, g) + c * kChunk + r * 16);
            }
        }
        // scales: 4 blocks x 128 columns (q8_0) or 128 columns once per group (q8_K)
        rx = make_float4(0.f, 0.f, 0.f, 0.f);
        if (tid < (KQ ? 32 : 128)) {
            const int blk = KQ ? 0 : tid >> 5, c4 = (tid & 31) * 4;
            const int64_t row = KQ ? g : (int64_t)s * 4 + blk;
            const float * src = p.dT + row * p.ldT + col0 + n0 + c4;
            if (n0 + c4 + 0 < p.N) rx.x = src[0];
            if (n0 + c4 + 1 < p.N) rx.y = src[1];
            if (n0 + c4 + 2 < p.N) rx.z = src[2];
            if (n0 + c4 + 3 < p.N) rx.w = src[3];
        }
    };
    auto store = [&](int buf) {
        uint8_t * A = lds + buf * kStage;
        uint8_t * B = A + kAB;
        float * X = reinterpret_cast<float *>(B + kBB);
#pragma unroll
        for (int q = 0; q < kNA; ++q) {
            const int u = tid + kT * q, c = u >> 3, un = u & 7;
            *reinterpret_cast<uint4 *>(A + c * kAP + un * 16) = ra[q];
        }
#pragma unroll
        for (int q = 0; q < kNB; ++q) {
            const int u = tid + kT * q;
            if (u < kBB / 16) *reinterpret_cast<uint4 *>(B + u * 16) = rb[q];
        }
        if (tid < (KQ ? 32 : 128)) *reinterpret_cast<float4 *>(X + tid * 4) = rx;
    };

    // ---- per-wave tile: image tile wr (64 rows = 2 MFMA row tiles) x columns wn * 32 .. + 32
    const int wr = wave & 1, wn = wave >> 1;
    const int h = lane >> 5, l32 = lane & 31;
    float out[2][16];
    v16i c1[2], c2[2], c3[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) out[rt][r] = 0.0f;
        c1[rt] = v16i{};
        c2[rt] = v16i{};
        c3[rt] = v16i{};
    }

    if (s0 < s1) {
        fetch(s0);
        store(0);
    }
    __syncthreads();
    for (int s = s0; s < s1; ++s) {                               // uniform over the work-group
        const int buf = (s - s0) & 1;
        if (s + 1 < s1) fetch(s + 1);
        const uint8_t * A = lds + buf * kStage;
        const uint8_t * B = A + kAB + wr * 5 * kChunk;            // this wave's image tile
        const float * X = reinterpret_cast<const float *>(A + kAB + kBB);
        const int hh = s & 1;
        uint4 hdr[2];                                             // the lane's row headers (chunk 8)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) hdr[rt] = *reinterpret_cast<const uint4 *>(B + 4 * kChunk + (32 * rt + l32) * 16);
#pragma unroll UQ
        for (int q = 0; q < 4; ++q) {
            const v4i a = *reinterpret_cast<const v4i *>(A + (wn * 32 + l32) * kAP + q * 32 + 16 * h);
            if constexpr (!KQ) {
                // Q4_0 block 4 hh + q: chunk slot q, low nibbles (k < 16) for h = 0, high for h = 1
                float dx[16];
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const float4 v = *reinterpret_cast<const float4 *>(X + q * kBN + wn * 32 + 8 * g4 + 4 * h);
                    dx[4 * g4] = v.x; dx[4 * g4 + 1] = v.y; dx[4 * g4 + 2] = v.z; dx[4 * g4 + 3] = v.w;
                }
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const uint4 v = *reinterpret_cast<const uint4 *>(B + q * kChunk + (32 * rt + l32) * 16);
                    const uint32_t e[4] = { v.x, v.y, v.z, v.w };
                    uint32_t o[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t nib = ((e[i] >> (4 * h)) & 0x0F0F0F0Fu) | 0x80808080u;
                        o[i] = (nib - 0x08080808u) ^ 0x80808080u;   // q - 8, bytewise
                    }
                    const v4i bq = v4i{ (int)o[0], (int)o[1], (int)o[2], (int)o[3] };
                    const int blk = 4 * hh + q;
                    const uint32_t hw = blk < 2 ? hdr[rt].x : blk < 4 ? hdr[rt].y : blk < 6 ? hdr[rt].z : hdr[rt].w;
                    const float dw = h2f(hw >> (16 * (blk & 1)));
                    const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, v16i{}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) out[rt][r] += (float)d[r] * (dw * dx[r]);
                }
            } else {
                // Q4_K sub-block jj = 4 hh + q: chunk slot 2 (q / 2) + h, low nibbles for even q
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const uint4 v = *reinterpret_cast<const uint4 *>(B + (2 * (q >> 1) + h) * kChunk + (32 * rt + l32) * 16);
                    const int jj = 4 * hh + q, b8 = 8 * (jj & 3);
                    uint32_t sc, mn;                              // get_scale_min_k4 (P01:2164-2176)
                    if (jj < 4) {
                        sc = (hdr[rt].y >> b8) & 63;
                        mn = (hdr[rt].z >> b8) & 63;
                    } else {
                        sc = ((hdr[rt].w >> b8) & 0xF) | (((hdr[rt].y >> b8) >> 6 & 3) << 4);
                        mn = ((hdr[rt].w >> b8) >> 4 & 0xF) | (((hdr[rt].z >> b8) >> 6 & 3) << 4);
                    }
                    const uint32_t sl = sc & 7u, sh = sc >> 3;
                    const uint32_t e[4] = { v.x, v.y, v.z, v.w };
                    uint32_t oh[4], ol[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t nib = (e[i] >> (4 * (q & 1))) & 0x0F0F0F0Fu;
                        oh[i] = v2_mul(nib, sh);
                        ol[i] = v2_mul(nib, sl);
                    }
                    const v4i bh = v4i{ (int)oh[0], (int)oh[1], (int)oh[2], (int)oh[3] };
                    const v4i bl = v4i{ (int)ol[0], (int)ol[1], (int)ol[2], (int)ol[3] };
                    const int mrep = (int)(mn * 0x01010101u);
                    const v4i bm = v4i{ mrep, mrep, mrep, mrep };
                    c1[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bh, c1[rt], 0, 0, 0);
                    c2[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bl, c2[rt], 0, 0, 0);
                    c3[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bm, c3[rt], 0, 0, 0);
                }
            }
        }
        if constexpr (KQ) {
            if (hh == 1) {                                        // end of the super-block (uniform)
                float dx[16];
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const float4 v = *reinterpret_cast<const float4 *>(X + wn * 32 + 8 * g4 + 4 * h);
                    dx[4 * g4] = v.x; dx[4 * g4 + 1] = v.y; dx[4 * g4 + 2] = v.z; dx[4 * g4 + 3] = v.w;
                }
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const float d = h2f(hdr[rt].x), dmin = h2f(hdr[rt].x >> 16);
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int isc = 8 * c1[rt][r] + c2[rt][r];
                        out[rt][r] += dx[r] * (d * (float)isc - dmin * (float)c3[rt][r]);
                    }
                    c1[rt] = v16i{};
                    c2[rt] = v16i{};
                    c3[rt] = v16i{};
                }
            }
        }
        if (s + 1 < s1) store(buf ^ 1);                           // the other buffer was last read a stage ago
        __syncthreads();
    }

    // ---- store: lane holds row 32 rt + l32 of its image tile for 16 columns
    float * dst = p.dst + i2 * p.bt.d_nb2 + i3 * p.bt.d_nb3;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const int64_t m = (2 * mtile + wr) * kTileRows + 32 * rt + l32;
        if (m >= p.w.M) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t n = n0 + wn * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (n < p.N) {
                float * o = dst + n * p.bt.d_nb1 + m;
                if (p.KS == 1) *o = out[rt][r];
                else atomicAdd(o, out[rt][r]);
            }
        }
    }
}

}  // namespace

bool gemm2_supported(int type) { return type == QMM_TYPE_Q4_0 || type == QMM_TYPE_Q4_K; }

// K split: enough work-groups to cover the chip (QMM_GEMM_WGS, default 512),
// whole groups per slice
static void g2_split(const WView & w, int64_t N, int64_t nbatch, int * KS, int * spk) {
    static const int64_t target = [] {
        const char * e = getenv("QMM_GEMM_WGS");
        return e ? std::max<int64_t>(1, atoll(e)) : (int64_t)512;
    }();
    const int64_t wgs = ((w.M + 127) / 128) * ((N + kBN - 1) / kBN) * nbatch;
    const int64_t ks = std::max<int64_t>(1, std::min<int64_t>(w.G, (target + wgs - 1) / wgs));
    const int64_t gps = (w.G + ks - 1) / ks;
    *spk = (int)(2 * gps);
    *KS = (int)((w.G + gps - 1) / gps);
}

int gemm2_kslices(const WView & w, int64_t N, int64_t nbatch) {
    int ks, spk;
    g2_split(w, N, nbatch, &ks, &spk);
    return ks;
}

void gemm2_shape(const WView & w, int64_t N, int64_t nbatch, int64_t * workgroups, int * threads, int * lds_bytes) {
    int ks, spk;
    g2_split(w, N, nbatch, &ks, &spk);
    *workgroups = ((w.M + 127) / 128) * ((N + kBN - 1) / kBN) * ks * nbatch;
    *threads = kT;
    *lds_bytes = 2 * kStage;
}

hipError_t launch_gemm2(int type, const WView & w, const ActBuf & a, int64_t N, int64_t nbatch, const GemmBatch & bt,
                        float * dst, hipStream_t s, const KTime * kt) {
    if (!gemm2_supported(type) || !a.dT || a.ldk != w.G * 256 || a.ldT < N * nbatch + 64 || N <= 0 || nbatch <= 0 ||
        nbatch > 65535 || a.vdt != vec_dot_type(type))
        return hipErrorInvalidValue;
    G2Params p{};
    p.w = w;
    p.xc = a.codes;
    p.ldk = a.ldk;
    p.dT = a.dT;
    p.ldT = a.ldT;
    p.N = N;
    p.mt = (w.M + 127) / 128;
    p.nt = (N + kBN - 1) / kBN;
    p.nst = 2 * w.G;
    g2_split(w, N, nbatch, &p.KS, &p.spk);
    p.bt = bt;
    p.dst = dst;
    const int64_t total = p.mt * p.nt * p.KS;
    p.chunk = (total + 7) / 8;
    const int64_t grid = p.chunk * 8;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 g((unsigned)grid, (unsigned)nbatch);
    const size_t lds = 2 * (size_t)kStage;
    if (type == QMM_TYPE_Q4_0) {
        if (kt) hipExtLaunchKernelGGL(k_gemm2<QMM_TYPE_Q4_0>, g, dim3(kT), (uint32_t)lds, s, kt->start, kt->stop, 0, p);
        else k_gemm2<QMM_TYPE_Q4_0><<<g, kT, lds, s>>>(p);
    } else {
        if (kt) hipExtLaunchKernelGGL(k_gemm2<QMM_TYPE_Q4_K>, g, dim3(kT), (uint32_t)lds, s, kt->start, kt->stop, 0, p);
        else k_gemm2<QMM_TYPE_Q4_K><<<g, kT, lds, s>>>(p);
    }
    return hipGetLastError();
}

}  // namespace qmm
