// k_gemm3.hip - prefill GEMM for the block types with one float scale per 32 weights (Q4_0,
// Q8_0, IQ4_NL) on gfx950 v_mfma_i32_32x32x32_i8, weights streamed by each wave.
//
// Role of the reference's int8 prefill GEMM (kernel_mul_mm_kq2d_q4_0_i8, P0099:377-455) and
// its fp16 tile kernel for Q8_0 (P02:4359-4384), redesigned for CDNA4 and for ggml-cpu's
// numerics.  ggml's dot for these types is sum_b d_x(b) d_w(b) I_b, a scale per 32-weight
// block on both sides, so every output takes a float multiply-add per block on top of the
// block's integer dot I_b: two VALU instructions per output and block, 32 per 32x32x32 MFMA.
// The VALU, not the MFMA, bounds this GEMM, so the design keeps the SIMDs' VALU issuing:
//  * a wave owns one 64-row tile of the weight image x one column tile of 32 over one K slice
//    and streams its weights itself: lane l loads row l's 16 bytes of a block (one coalesced
//    1 KB buffer load of the image's chunk plane), unpacks them in registers and trades
//    halves with v_permlane32_swap into the B operands of rows 0-31 and rows 32-63;
//  * the activations come from the pre-pass in MFMA A-operand order (1 KB per column tile and
//    block) with their scales as f32 in MFMA output order; the kU waves of a work-group that
//    share a K slice (different row tiles, same columns) stage them in LDS once, a stage of
//    blocks ahead, one barrier per stage;
//  * Q4_0 codes are unpacked into the high nibble of each byte after flipping bit 3: the int8
//    byte (q ^ 8) << 4 is 16 (q - 8), with no borrow handling; the sums carry the factor 16,
//    taken off exactly (a power of two) at the store;
//  * the MFMA's C input is the bits of the float 12582912 (1.5 * 2^23), so its int32 result
//    read as a float is 12582912 + I exactly; fma(that, d_w, -12582912 d_w) is I d_w rounded
//    once and fma(., d_x, acc) accumulates it: two plain f32 FMAs per output and block (on
//    gfx950 an fp16 source operand, v_fma_mix, halves the FMA issue rate);
//  * three waves per SIMD (at most 168 registers): work-groups of kU = 4 waves when the tiles
//    fill the chip, three of them per CU, else work-groups of 3 K slices x kU (12 waves, one
//    per CU: a work-group's waves go to the CU's SIMDs in turn, so 8-wave groups would leave
//    room for one group only and 2 waves per SIMD);
//  * the K slices of a row tile are waves of one work-group: slices 1.. add their sums into LDS
//    at the end and slice 0 stores, so dst is written once (non-temporal), with no atomics and
//    no zeroing;
//  * every load goes through a buffer resource: the wave-uniform address math stays on the
//    SALU, and reads past a resource's range (the last stage of a row whose groups are not a
//    whole number of stages) return zeros;
//  * work-groups that share weight rows are numbered onto one XCD (work-group b runs on XCD
//    b % 8), so a row tile's weights come from HBM once and from that XCD's L2 after.
// MFMA layouts (i = lane % 32, h = lane / 32): A operand lane (i, h) = column i, k 16 h..+15;
// B operand lane (j, h) = row j, k 16 h..+15; result register r of lane (j, h) = column
// 8 (r / 4) + 4 h + r % 4 of row j.
#include "qmm_device.h"

#include <hip/hip_ext.h>

#include <algorithm>
#include <cstdlib>

namespace qmm {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kMagic = 0x4B400000;       // float 12582912: its bits + i are the float 12582912 + i, |i| < 2^22
constexpr int kU = 4;                    // row tiles per work-group: the waves sharing a K slice's staging
constexpr int kMaxKS = 3;                // K slices per work-group (12 waves: 3 per SIMD)
constexpr int kRing = 2;                 // weight blocks in flight per wave
// blocks per stage: two groups, one for Q8_0 (its two code chunks per block take the registers);
// a stage in LDS holds the A operands of its blocks (1 KB each), then their f32 scales (128 B)
__host__ __device__ constexpr int stage_blocks(int type) { return type == QMM_TYPE_Q8_0 ? 8 : 16; }
__host__ __device__ constexpr int stage_bytes(int type) { return stage_blocks(type) * (1024 + 128); }

struct G3Params {
    WView w;
    const int8_t * tA;
    const float * tD;
    int64_t nblk;                        // blocks per activation column
    int64_t ntb;                         // column tiles per batch
    int64_t N;                           // columns per batch
    int64_t mbn, nbn;                    // work-group blocks per batch along M (kU row tiles) and N (C column tiles)
    int64_t total;                       // mbn * nbn
    int64_t chunk;                       // ceil(total / 8): logical work-groups per XCD
    int KS, sps, nst;                    // K slices, stages per slice, stages along K (kSB blocks each)
    GemmBatch bt;
    float * dst;
};

// lo (k 0..15) and hi (k 16..31) of the lane's own row -> B operands of rows 0-31 (op0) and
// rows 32-63 (op1): lanes 32-63 trade their lo for lanes 0-31's hi
__device__ __forceinline__ void swap_halves(const uint4 & lo, const uint4 & hi, v4i & op0, v4i & op1) {
    const auto a = __builtin_amdgcn_permlane32_swap(lo.x, hi.x, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(lo.y, hi.y, false, false);
    const auto c = __builtin_amdgcn_permlane32_swap(lo.z, hi.z, false, false);
    const auto d = __builtin_amdgcn_permlane32_swap(lo.w, hi.w, false, false);
    op0 = v4i{ (int)a[0], (int)b[0], (int)c[0], (int)d[0] };
    op1 = v4i{ (int)a[1], (int)b[1], (int)c[1], (int)d[1] };
}

// a per-row value of the lane's own row -> that of row lane % 32 (r0) and row 32 + lane % 32 (r1)
__device__ __forceinline__ void swap_rows(uint32_t v, uint32_t & r0, uint32_t & r1) {
    const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    r0 = a[0];
    r1 = a[1];
}

// Buffer loads: a wave-uniform resource (base and byte size in scalar registers), a 32-bit lane
// offset and a scalar block offset, so the per-load address math stays on the SALU; reads past
// the size return zeros.  (Word 3 is the gfx9 raw-buffer format.)
typedef unsigned v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void * base, uint32_t bytes) {
    const uint64_t v = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(((uint64_t)hi << 32) | lo), 0,
                                             (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
__device__ __forceinline__ uint4 bld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t bld4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}

// one weight block of the lane's row in flight
template <int TYPE> struct WBlk {
    uint4 c[TYPE == QMM_TYPE_Q8_0 ? 2 : 1];   // codes: Q8_0 qs[0:16], qs[16:32]; else the 16 bytes of qs
    uint32_t d;                               // the dword of the d plane holding the block's fp16 scale
};

template <int TYPE>
__global__ __launch_bounds__(64 * kU * kMaxKS) void k_gemm3(G3Params p) {
    constexpr bool Q8 = TYPE == QMM_TYPE_Q8_0;
    constexpr bool NLQ = TYPE == QMM_TYPE_IQ4_NL;
    constexpr int kDch = Q8 ? 16 : 8;                         // chunk plane of the block scales
    constexpr int kSB = stage_blocks(TYPE), kSA = kSB * 1024, kStage = stage_bytes(TYPE);
    static_assert(kSB % kRing == 0 && kSB % kU == 0, "ring slots repeat every stage; A blocks spread over the waves");
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int u = wave % kU, ks = wave / kU;

    const uint32_t L = (blockIdx.x & 7) * (uint32_t)p.chunk + (blockIdx.x >> 3);
    if (L >= (uint32_t)p.total) return;                       // uniform over the work-group
    const uint32_t mb = L / (uint32_t)p.nbn, nb = L - mb * (uint32_t)p.nbn;
    const uint32_t bz = blockIdx.y;
    const uint32_t i2 = bz % (uint32_t)p.bt.ne12, i3 = bz / (uint32_t)p.bt.ne12;
    const int64_t mat = (int64_t)(i2 / (uint32_t)p.bt.r2) + (int64_t)(i3 / (uint32_t)p.bt.r3) * p.bt.ne02;
    const int64_t mt_raw = (int64_t)mb * kU + u;
    const bool row_ok = mt_raw < p.w.ntiles;                  // a missing tile computes a copy, stores nothing
    const int64_t mtile = row_ok ? mt_raw : p.w.ntiles - 1;
    const int64_t ctile = (int64_t)bz * p.ntb + nb;           // the work-group's column tile
    // this slice's stages [s0, s1); every slice runs sps iterations (the barriers are work-group
    // wide), the idle ones past s1 only staging (clamped) and waiting
    const int s0 = ks * p.sps;
    const int s1 = std::min(s0 + p.sps, p.nst);
    const int slast = s1 - 1;                                 // (every slice has stages: KS = ceil(nst / sps))
    const int kb_last = s1 * kSB - 1;                         // (blocks past the row read zeros: buffer ranges)

    // ---- buffer resources (wave-uniform): the tile's weight row, the column tile's A operands
    // (1 KB per block) and f32 scales (128 B per block)
    const __amdgpu_buffer_rsrc_t wbuf = buffer_rsrc(tile_group(p.w, mat, mtile, 0), (uint32_t)(p.w.G * p.w.tg));
    const __amdgpu_buffer_rsrc_t abuf = buffer_rsrc(p.tA + ctile * p.nblk * 1024, (uint32_t)(p.nblk * 1024));
    const __amdgpu_buffer_rsrc_t dbuf = buffer_rsrc(p.tD + ctile * p.nblk * 32, (uint32_t)(p.nblk * 128));
    const uint32_t lane16 = (uint32_t)lane * 16;
    const uint32_t tgs = (uint32_t)p.w.tg;

    // ---- staging: the kU waves of a slice copy a stage (kSB blocks of A and scales) into LDS,
    // wave u the A operands of blocks u, u + kU, ... and 16-byte units u * 16 + lane (lane < 16)
    // of the scales
    constexpr int kNA = kSB / kU;
    uint4 ra[kNA], rd = make_uint4(0, 0, 0, 0);
    const bool dlane = lane < kSB * 8 / kU;
    auto fetch = [&](int st) {
        st = std::min(st, slast);
#pragma unroll
        for (int j = 0; j < kNA; ++j) ra[j] = bld16(abuf, lane16, (uint32_t)(st * kSB + u + kU * j) * 1024);
        if (dlane) rd = bld16(dbuf, (uint32_t)(u * (kSB * 8 / kU) + lane) * 16, (uint32_t)st * kSB * 128);
    };
    auto store = [&](int buf) {
        uint8_t * S = lds + (ks * 2 + buf) * kStage;
#pragma unroll
        for (int j = 0; j < kNA; ++j) *reinterpret_cast<uint4 *>(S + (u + kU * j) * 1024 + lane16) = ra[j];
        if (dlane) *reinterpret_cast<uint4 *>(S + kSA + (u * (kSB * 8 / kU) + lane) * 16) = rd;
    };

    // ---- weight ring: block kb of the K axis, clamped to the slice's last block
    WBlk<TYPE> ring[kRing];
    auto wload = [&](WBlk<TYPE> & r, int kb) {
        kb = std::min(kb, kb_last);
        const uint32_t pl = (uint32_t)kb & 7, tg = (uint32_t)(kb >> 3) * tgs;   // uniform
        r.c[0] = bld16(wbuf, lane16, tg + pl * (Q8 ? 2 : 1) * kChunk);
        if constexpr (Q8) r.c[1] = bld16(wbuf, lane16, tg + (2 * pl + 1) * kChunk);
        r.d = bld4(wbuf, lane16, tg + kDch * kChunk + 4 * (pl >> 1));
    };

    v16f acc0 = v16f{}, acc1 = v16f{};                       // rows lane % 32 and 32 + lane % 32
    v16i magic;
#pragma unroll
    for (int r = 0; r < 16; ++r) magic[r] = kMagic;
    struct Act {
        v4i a;                                                // A operand
        float dx[16];                                         // scales of the lane's 16 result columns
    };
    auto aread = [&](Act & x, const uint8_t * S, int j) {     // block j of a stage in LDS
        x.a = *reinterpret_cast<const v4i *>(S + j * 1024 + lane16);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = *reinterpret_cast<const float4 *>(S + kSA + j * 128 + h * 64 + 16 * q);
            x.dx[4 * q] = v.x;
            x.dx[4 * q + 1] = v.y;
            x.dx[4 * q + 2] = v.z;
            x.dx[4 * q + 3] = v.w;
        }
    };
    // acc += (I d_w rounded once) d_x for the 16 results of one MFMA: the 16 products first (in the
    // result's registers), then the 16 accumulations, so no VALU instruction waits on the one just
    // before it; plain f32 FMAs (an fp16 source operand halves their issue rate)
    auto consume = [&](v16f & acc, const v16i & e, float dw, float nm, const float (&dx)[16]) {
        v16f tv;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int iv = e[r];
            tv[r] = __builtin_fmaf(__builtin_bit_cast(float, iv), dw, nm);
        }
        asm volatile("" : "+v"(tv));
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = __builtin_fmaf(tv[r], dx[r], acc[r]);
    };
    auto compute = [&](int buf, int st) {
        const uint8_t * S = lds + (ks * 2 + buf) * kStage;
        Act x;
#pragma unroll
        for (int j = 0; j < kSB; ++j) {
            const int kb = st * kSB + j;
            aread(x, S, j);                                   // (the SIMD's other waves cover the LDS latency)
            WBlk<TYPE> & wb = ring[j % kRing];
            // block kb's weights of the lane's row -> B operands of rows 0-31 and 32-63, and d_w of the
            // output rows lane % 32 and 32 + lane % 32
            uint4 lo, hi;
            if constexpr (Q8) {
                lo = wb.c[0];
                hi = wb.c[1];
            } else if constexpr (NLQ) {
                const uint4 q = wb.c[0];
                lo = make_uint4(iq4_lookup(q.x & 0x0F0F0F0Fu), iq4_lookup(q.y & 0x0F0F0F0Fu),
                                iq4_lookup(q.z & 0x0F0F0F0Fu), iq4_lookup(q.w & 0x0F0F0F0Fu));
                hi = make_uint4(iq4_lookup((q.x >> 4) & 0x0F0F0F0Fu), iq4_lookup((q.y >> 4) & 0x0F0F0F0Fu),
                                iq4_lookup((q.z >> 4) & 0x0F0F0F0Fu), iq4_lookup((q.w >> 4) & 0x0F0F0F0Fu));
            } else {
                // (q ^ 8) in the high nibble: the int8 byte is 16 (q - 8)
                const uint32_t x0 = wb.c[0].x ^ 0x88888888u, x1 = wb.c[0].y ^ 0x88888888u;
                const uint32_t x2 = wb.c[0].z ^ 0x88888888u, x3 = wb.c[0].w ^ 0x88888888u;
                lo = make_uint4((x0 << 4) & 0xF0F0F0F0u, (x1 << 4) & 0xF0F0F0F0u, (x2 << 4) & 0xF0F0F0F0u,
                                (x3 << 4) & 0xF0F0F0F0u);
                hi = make_uint4(x0 & 0xF0F0F0F0u, x1 & 0xF0F0F0F0u, x2 & 0xF0F0F0F0u, x3 & 0xF0F0F0F0u);
            }
            v4i op0, op1;
            swap_halves(lo, hi, op0, op1);
            uint32_t d0b, d1b;
            swap_rows(wb.d >> (16 * (kb & 1)), d0b, d1b);
            wload(wb, kb + kRing);                            // the slot's next block
            float dw0 = h2f(d0b), dw1 = h2f(d1b);
            asm volatile("" : "+v"(dw0), "+v"(dw1));          // f32 operands (no fp16 source folding)
            if (QMM_RED == 6) dw1 = dw0;                      // (mutation 6: rows 32-63 take rows 0-31's scale)
            const float nm0 = -12582912.0f * dw0, nm1 = -12582912.0f * dw1;
            const Act & c = x;
            // (one MFMA result at a time: the SIMD's other waves cover its latency)
            const v16i e0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(c.a, op0, magic, 0, 0, 0);
            consume(acc0, e0, dw0, nm0, c.dx);
            __builtin_amdgcn_sched_barrier(0);
            const v16i e1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(c.a, op1, magic, 0, 0, 0);
            consume(acc1, e1, dw1, nm1, c.dx);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // ---- K loop: stage s + 1 is in registers while s is computed; it goes to the other buffer,
    // whose stage s - 1 every wave finished before the last barrier
#pragma unroll
    for (int i = 0; i < kRing; ++i) wload(ring[i], s0 * kSB + i);
    fetch(s0);
    store(0);
    fetch(s0 + 1);
    __syncthreads();
    for (int it = 0; it < p.sps; ++it) {                      // uniform over the work-group
        if (s0 + it < s1) compute(it & 1, s0 + it);
        if (it + 1 < p.sps) store((it + 1) & 1);
        if (it + 2 < p.sps) fetch(s0 + it + 2);
        __syncthreads();
    }

    // ---- K slices 1.. add their sums into slice 0's through LDS (fixed order), slice 0 stores
    if (p.KS > 1) {
        float * red = reinterpret_cast<float *>(lds);
        if (ks > 0) {
            float * o = red + ((size_t)((ks - 1) * kU + u) * 32) * 64 + lane;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                o[r * 64] = acc0[r];
                o[(16 + r) * 64] = acc1[r];
            }
        }
        __syncthreads();
        if (ks > 0) return;
        for (int k = 1; k < p.KS; ++k) {
            const float * o = red + ((size_t)((k - 1) * kU + u) * 32) * 64 + lane;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc0[r] += o[r * 64];
                acc1[r] += o[(16 + r) * 64];
            }
        }
    }
    if (!row_ok) return;
    const float scale = (TYPE == QMM_TYPE_Q4_0) ? 0.0625f : 1.0f;   // Q4_0 codes carried 16 (q - 8)
    float * dst = p.dst + (int64_t)i2 * p.bt.d_nb2 + (int64_t)i3 * p.bt.d_nb3;
    const int64_t n0 = (int64_t)nb * 32;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int64_t m = mtile * kTileRows + 32 * t + (lane & 31);
        if (m >= p.w.M) continue;
        const v16f & v = t ? acc1 : acc0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t n = n0 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (n < p.N) __builtin_nontemporal_store(v[r] * scale, dst + n * p.bt.d_nb1 + m);
        }
    }
}

template <int TYPE>
hipError_t launch_t(const G3Params & p, const G3Shape & sh, const dim3 & g, hipStream_t s, const KTime * kt) {
    static const hipError_t attr =
        hipFuncSetAttribute((const void *)k_gemm3<TYPE>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    const dim3 b(sh.threads);
    if (kt) hipExtLaunchKernelGGL(k_gemm3<TYPE>, g, b, (uint32_t)sh.lds, s, kt->start, kt->stop, 0, p);
    else k_gemm3<TYPE><<<g, b, sh.lds, s>>>(p);
    return hipGetLastError();
}

int env_int3(const char * name, int dflt) {
    const char * e = getenv(name);
    return e ? atoi(e) : dflt;
}

}  // namespace

bool gemm3_supported(int type) {
    static const bool on = env_int3("QMM_GEMM3", 1) != 0;
    return on && (type == QMM_TYPE_Q4_0 || type == QMM_TYPE_Q8_0 || type == QMM_TYPE_IQ4_NL);
}

// Launch shape: C column tiles per wave (2 shares each weight unpack between two column tiles,
// at twice the accumulators), kU row tiles per work-group, and K slices so that the waves come
// to about `target` (3 per SIMD).
bool gemm3_shape(int type, const WView & w, int64_t N, int64_t nbatch, G3Shape * sh) {
    if (!gemm3_supported(type) || N <= 0 || nbatch <= 0 || nbatch > 65535 || w.G <= 0 || w.ntiles <= 0) return false;
    const int64_t ntb = (N + 31) / 32;
    sh->C = 1;
    sh->U = kU;
    sh->SB = stage_blocks(type);
    sh->mbn = (w.ntiles + kU - 1) / kU;
    sh->nbn = ntb;
    sh->nst = (int)((w.G * 8 + sh->SB - 1) / sh->SB);
    // Work-groups of kU waves (one per SIMD, three per CU) when that fills the chip, else of 3 K
    // slices (12 waves: three per SIMD in one work-group); the waves of a work-group are spread
    // over the CU's SIMDs in turn, so 8-wave groups would leave room for one group only.
    const int64_t units = sh->mbn * sh->nbn * nbatch;             // work-groups of one K slice
    int ks = units * kU >= 2048 ? 1 : kMaxKS;
    const int ksenv = env_int3("QMM_GEMM3_KS", 0);
    if (ksenv >= 1 && ksenv <= kMaxKS) ks = ksenv;
    ks = std::min(ks, sh->nst);
    sh->sps = (sh->nst + ks - 1) / ks;
    sh->KS = (sh->nst + sh->sps - 1) / sh->sps;                   // no slice without stages
    sh->threads = 64 * kU * sh->KS;
    sh->lds = std::max(sh->KS * 2 * stage_bytes(type), (sh->KS - 1) * kU * 32 * 64 * 4);
    sh->workgroups = 8 * ((units / nbatch + 7) / 8) * nbatch;
    return units / nbatch < 0x7fffffff && sh->lds <= 160 * 1024;
}

hipError_t launch_gemm3(int type, const WView & w, const TiledAct & a, int64_t nbatch, const GemmBatch & bt,
                        float * dst, hipStream_t s, const KTime * kt) {
    G3Shape sh;
    if (!gemm3_shape(type, w, a.N, nbatch, &sh) || !a.A || !a.D || a.nblk != w.G * 8 || a.ntb != (a.N + 31) / 32 ||
        a.ntiles != a.ntb * nbatch)
        return hipErrorInvalidValue;
    G3Params p{};
    p.w = w;
    p.tA = a.A;
    p.tD = a.D;
    p.nblk = a.nblk;
    p.ntb = a.ntb;
    p.N = a.N;
    p.mbn = sh.mbn;
    p.nbn = sh.nbn;
    p.total = sh.mbn * sh.nbn;
    p.chunk = (p.total + 7) / 8;
    p.KS = sh.KS;
    p.sps = sh.sps;
    p.nst = sh.nst;
    p.bt = bt;
    p.dst = dst;
    const dim3 g((unsigned)(8 * p.chunk), (unsigned)nbatch);
    switch (type) {
        case QMM_TYPE_Q4_0: return launch_t<QMM_TYPE_Q4_0>(p, sh, g, s, kt);
        case QMM_TYPE_Q8_0: return launch_t<QMM_TYPE_Q8_0>(p, sh, g, s, kt);
        case QMM_TYPE_IQ4_NL: return launch_t<QMM_TYPE_IQ4_NL>(p, sh, g, s, kt);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
