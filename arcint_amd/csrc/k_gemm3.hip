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

// ---- Q4_K ------------------------------------------------------------------------------------
// Role of the reference's K-quant integer GEMM (P01:1919-2024: an integer dot per sub-block, its
// 6-bit scale applied to the dot, the min term once per super-block), on q8_K activations.
//  * a wave owns 32 rows (one half of a 64-row image tile) x 64 columns (two column tiles) over
//    one K slice: lane (j, h) loads chunk plane 2c + h of row j, whose low nibbles are k
//    16 h .. 16 h + 15 of sub-block 2c and whose high nibbles are those of sub-block 2c + 1, which
//    is the MFMA's B operand for row j as it lies (no lane exchange), and the output lane (j, h)
//    holds row j, so the lane's own header gives its row's scales;
//  * the 6-bit sub-block scale goes into the B operand: sc = 8 sh + sl with 3-bit halves, so
//    q sh and q sl (<= 105) are int8 (one packed 16-bit multiply per dword: a byte times s <= 7
//    carries nothing into the next), and four MFMA chains per sub-block (sh and sl, two column
//    tiles) accumulate the super-block's sums in place; isc = 8 sum_sh + sum_sl at the end.  The
//    VALU never waits for an MFMA result inside the super-block (a per-row multiply-add on each
//    sub-block's int32 result cost 256 VALU instructions per super-block and wave, 47 % of it);
//  * the min term sum_j m_j bsum_j is two MFMAs per column tile and super-block: A = the
//    columns' split sums bh (then bl, bsum = 64 bh + bl) at k = j, B = the row's 8 mins; the
//    second one starts from 64 * first + the bits of 12582912.0f, so its result read as a float
//    is 12582912 + the exact min sum (|sum| < 2^22) and one FMA takes dmin times it;
//  * per super-block and output: out += dx * (d * isc - dmin * imn);
//  * activations (the super-block's A operands of both tiles, split sums and scales: 18 KB) go
//    from the pre-pass layout into LDS by buffer loads that write LDS directly (no registers), one
//    super-block ahead; the U row-half waves of a K slice share them, one barrier per super-block;
//  * the weights stream through registers one super-block ahead: a chunk is reloaded with the
//    next super-block's as soon as its two sub-blocks are done.
constexpr int kKQStage = 18 * 1024;           // A [2 tiles][8 sub-blocks][1 KB], S [2][32][16], D [2][32] f32 (1 KB slot)
constexpr int kKQMaxWaves = 12;
// every wave stages ceil(18 / U) units of 1 KB per super-block, the same count on every wave and
// every iteration (so the barrier waits for exactly these loads, not the weight loads issued
// after them); units past 18 read nothing (out of range) into a 1 KB slot after the stages
__host__ __device__ constexpr int kq_units(int U) { return (18 + U - 1) / U; }
// s_waitcnt immediate (gfx9 encoding): vmcnt 5 (bits 3:0, 15:14), expcnt and lgkmcnt not waited on
constexpr int kVmcnt5 = 5 | (0x7 << 4) | (0xF << 8);

struct KQParams {
    WView w;
    const int8_t * tA;
    const float * tD;
    const int8_t * tS;
    int64_t nsb;                         // super-blocks per column (the weights' groups)
    int64_t ntb;                         // column tiles per batch
    int64_t N;                           // columns per batch
    int64_t mbn, nbn;                    // work-group blocks per batch: U row halves along M, column pairs along N
    int64_t total, chunk;                // mbn * nbn, ceil(total / 8)
    int U, KS, sps;                      // row-half waves per K slice, K slices, super-blocks per slice
    GemmBatch bt;
    float * dst;
    // grouped MoE mode: work-group column pair nb is unit nb of the route (nbn = the units'
    // upper bound, *nunits the count), its activations gathered from the route's quantization
    const GemmUnit * units;
    const int32_t * nunits;
    const int8_t * codes;                // [column][ldk]
    const float * dcol;                  // [column][nsb]
    const int8_t * bsp;                  // [super-block][ldT][16]
    int64_t ldk, ldT, ncols;
};

// the two 16-bit halves of v times those of s (v_pk_mul_lo_u16)
__device__ __forceinline__ uint32_t mul_u16x2(uint32_t v, uint32_t s) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, v) * __builtin_bit_cast(u16x2, s));
}

// 4 bytes per lane from a buffer into LDS at lds + 4 lane (lds wave-uniform)
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint8_t * lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 4, (int)voff, (int)soff,
                                             0, 0);
}

// 16 bytes per lane from a buffer into LDS at lds + 16 lane (lds wave-uniform)
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t * lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, (int)voff, (int)soff,
                                             0, 0);
}

template <int U, bool GATHER>
__global__ __launch_bounds__(64 * kKQMaxWaves) void k_gemm3_q4k(KQParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, j32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int u = wave % U, ks = wave / U;

    const uint32_t L = (blockIdx.x & 7) * (uint32_t)p.chunk + (blockIdx.x >> 3);
    if (L >= (uint32_t)p.total) return;                       // uniform over the work-group
    const uint32_t mb = L / (uint32_t)p.nbn, nb = L - mb * (uint32_t)p.nbn;
    const uint32_t bz = blockIdx.y;
    const uint32_t i2 = bz % (uint32_t)p.bt.ne12, i3 = bz / (uint32_t)p.bt.ne12;
    int64_t mat = (int64_t)(i2 / (uint32_t)p.bt.r2) + (int64_t)(i3 / (uint32_t)p.bt.r3) * p.bt.ne02;
    int ncu = 64;                                             // grouped mode: the unit's columns
    if constexpr (GATHER) {
        if ((int32_t)nb >= __builtin_amdgcn_readfirstlane(*p.nunits)) return;   // uniform: past the route's units
        mat = __builtin_amdgcn_readfirstlane(p.units[nb].mat);
        ncu = __builtin_amdgcn_readfirstlane(p.units[nb].ncols);
    }
    const int64_t rh_raw = (int64_t)mb * U + u;               // the wave's row half
    const bool row_ok = rh_raw < 2 * p.w.ntiles;              // a missing row half computes a copy, stores nothing
    const int64_t rh = row_ok ? rh_raw : 2 * p.w.ntiles - 1;
    const int64_t mtile = rh >> 1;
    const int t = (int)(rh & 1);
    const int64_t ct0 = (int64_t)bz * p.ntb + 2 * (int64_t)nb; // the pair's first column tile
    const int64_t nct = std::min<int64_t>(2, p.ntb - 2 * (int64_t)nb);
    const int nsb = (int)p.nsb;
    const int s0 = ks * p.sps;
    const int s1 = std::min(s0 + p.sps, nsb);                 // (every slice has super-blocks)

    if (GATHER && mat < 0) {                                  // invalid ids: zero rows (uniform)
        const int64_t m = mtile * kTileRows + 32 * t + j32;
        if (!row_ok || m >= p.w.M || ks > 0) return;
        for (int n = h; n < ncu; n += 2) p.dst[p.units[nb].dst_off[n] + m] = 0.0f;
        return;
    }

    const __amdgpu_buffer_rsrc_t wbuf = buffer_rsrc(tile_group(p.w, mat, mtile, 0), (uint32_t)(p.w.G * p.w.tg));
    // the pair's activations; a pair with one tile reads zeros for the second (past the range);
    // grouped mode: the whole quantization, each lane at its own column (zeros past the unit)
    const __amdgpu_buffer_rsrc_t abuf = GATHER ? buffer_rsrc(p.codes, (uint32_t)(p.ncols * p.ldk))
                                               : buffer_rsrc(p.tA + ct0 * p.nsb * 8192, (uint32_t)(nct * p.nsb * 8192));
    const __amdgpu_buffer_rsrc_t sbuf = GATHER ? buffer_rsrc(p.bsp, (uint32_t)(p.nsb * p.ldT * 16))
                                               : buffer_rsrc(p.tS + ct0 * p.nsb * 512, (uint32_t)(nct * p.nsb * 512));
    const __amdgpu_buffer_rsrc_t dbuf = GATHER ? buffer_rsrc(p.dcol, (uint32_t)(p.ncols * p.nsb * 4))
                                               : buffer_rsrc(p.tD + ct0 * p.nsb * 32, (uint32_t)(nct * p.nsb * 128));
    const uint32_t lane16 = (uint32_t)lane * 16;
    // grouped mode: the activation column of lane (j32, h) in tile c (both lane halves share it),
    // and the column of lane `lane` for the S and D gathers (tile lane / 32); kOut past the unit
    constexpr uint32_t kOut = 0x7ff00000u;
    uint32_t gcol[2] = { 0, 0 }, gsd = 0;
    if constexpr (GATHER) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int slot = 32 * c + j32;
            gcol[c] = slot < ncu ? (uint32_t)p.units[nb].col[slot] : kOut;
        }
        gsd = (lane >> 5) ? gcol[1] : gcol[0];
    }

    // ---- staging of super-block s into buffer b of the slice: 18 units of 1 KB (A: tile
    // unit / 8, sub-block unit % 8; S; D, lanes 16.. reading zeros into the slot's padding),
    // wave u taking units u, u + U, ...
    constexpr int NU = kq_units(U);
    const uint32_t a_stride = (uint32_t)p.nsb * 8192, s_stride = (uint32_t)p.nsb * 512, d_stride = (uint32_t)p.nsb * 128;
    uint32_t s_lane = (uint32_t)(lane >> 5) * s_stride + (uint32_t)j32 * 16;
    uint32_t d_lane = lane < 16 ? (uint32_t)(lane >> 3) * d_stride + (uint32_t)(lane & 7) * 16 : kOut;
    // Grouped mode, A: unit (c, g) holds columns 4g..4g+3 of tile c whole (the super-block's 256
    // code bytes of each, 16 lanes per column: a few whole lines per load instead of 32 pieces);
    // in LDS column i of tile c sits at c 8192 + 256 i with its 16-byte chunk q at slot
    // q ^ (i & 15), so the MFMA operand reads (chunk 2 j + h of column i for lane (i, h)) hit
    // 16 different slots per 16 lanes: no bank conflicts.  avo[k]: lane offset of this wave's
    // k-th A unit.  S: the column's 16 bytes; D: its 4.
    uint32_t avo[NU];
#pragma unroll
    for (int k = 0; k < NU; ++k) avo[k] = 0;
    if constexpr (GATHER) {
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            const int unit = u + k * U;
            if (unit < 16) {
                const int ci = 4 * (unit & 7) + (lane >> 4);  // column of the tile
                const int slot = 32 * (unit >> 3) + ci;
                const uint32_t col = slot < ncu ? (uint32_t)p.units[nb].col[slot] : kOut;
                const uint32_t q = (uint32_t)((lane & 15) ^ (ci & 15));
                avo[k] = col == kOut ? kOut : col * (uint32_t)p.ldk + 16 * q;
            }
        }
        s_lane = gsd == kOut ? kOut : gsd * 16;
        d_lane = gsd == kOut ? kOut : gsd * (uint32_t)p.nsb * 4;
    }
    uint8_t * const dump = lds + 2 * p.KS * kKQStage;
    auto stage = [&](int s, int b) {
        uint8_t * S = lds + (ks * 2 + b) * kKQStage;
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            const int unit = u + i * U;                       // wave-uniform
            if (unit < 16) {
                if (GATHER)
                    dma16(abuf, S + unit * 1024, avo[i], (uint32_t)s * 256);
                else
                    dma16(abuf, S + unit * 1024, lane16 + (uint32_t)(unit >> 3) * a_stride + (uint32_t)(unit & 7) * 1024,
                          (uint32_t)s * 8192);
            } else if (unit == 16) {
                dma16(sbuf, S + 16 * 1024, s_lane, GATHER ? (uint32_t)(s * p.ldT * 16) : (uint32_t)s * 512);
            } else if (unit == 17) {
                if (GATHER) dma4(dbuf, S + 17 * 1024, d_lane, (uint32_t)s * 4);   // [tile][32] f32 in column order
                else dma16(dbuf, S + 17 * 1024, d_lane, (uint32_t)s * 128);
            } else {
                dma16(dbuf, dump, kOut, 0);                   // (nothing: keeps the count)
            }
        }
    };

    // ---- weights of the lane's row (32 t + j32): chunk planes 2c + h, and the header plane
    const uint32_t row16 = (uint32_t)(32 * t + j32) * 16, wl = row16 + (uint32_t)h * kChunk;
    const uint32_t tgs = (uint32_t)p.w.tg;
    uint4 ch[4], hd;

    v16f out0 = v16f{}, out1 = v16f{};                       // column tiles 0 and 1 of the pair
    auto compute = [&](int b, int s) {
        const uint8_t * S = lds + (ks * 2 + b) * kKQStage;
        // the row's 6-bit scales and mins (get_scale_min_k4, P01:2164-2176), four per word
        const uint32_t sc03 = hd.y & 0x3f3f3f3fu, mn03 = hd.z & 0x3f3f3f3fu;
        const uint32_t sc47 = (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u);
        const uint32_t mn47 = ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u);
        const uint32_t dd = hd.x;
        const uint32_t sn = (uint32_t)std::min(s + 1, s1 - 1) * tgs;   // the next super-block (clamped)
        hd = bld16(wbuf, row16, sn + 8 * kChunk);
        const uint32_t sh03 = (sc03 >> 3) & 0x07070707u, sl03 = sc03 & 0x07070707u;
        const uint32_t sh47 = (sc47 >> 3) & 0x07070707u, sl47 = sc47 & 0x07070707u;
        v16i acc[4];                                          // [sh, sl] x [tile 0, tile 1]
        // the A operands of sub-block j of both column tiles, read one sub-block ahead (the LDS
        // latency runs under the previous sub-block's MFMAs)
        auto aread = [&](int j, v4i & x0, v4i & x1) {
            // (grouped mode: chunk 2 j + h of column j32 at its swizzled slot)
            const uint32_t aoff = GATHER ? (uint32_t)j32 * 256 + 16 * (uint32_t)((2 * j + h) ^ (j32 & 15))
                                         : (uint32_t)(j * 1024) + lane16;
            x0 = *reinterpret_cast<const v4i *>(S + aoff);
            x1 = *reinterpret_cast<const v4i *>(S + 8192 + aoff);
        };
        v4i na0, na1;
        aread(0, na0, na1);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint4 q = ch[j >> 1];
            const int nsh = 4 * (j & 1);
            const uint32_t n0 = (q.x >> nsh) & 0x0F0F0F0Fu, n1 = (q.y >> nsh) & 0x0F0F0F0Fu;
            const uint32_t n2 = (q.z >> nsh) & 0x0F0F0F0Fu, n3 = (q.w >> nsh) & 0x0F0F0F0Fu;
            if (j & 1) ch[j >> 1] = bld16(wbuf, wl, sn + 2 * (j >> 1) * kChunk);
            const v4i a0 = na0, a1 = na1;
            if (j < 7) aread(j + 1, na0, na1);
            const int js = j ^ (QMM_RED == 5);                // (mutation 5: neighbouring scales swapped)
            // the sub-block's sh and sl in both 16-bit halves (bytes 1 and 3 zero)
            const uint32_t sel = 0x0c000c00u | (uint32_t)(js & 3) * 0x00010001u;
            const uint32_t mh = __builtin_amdgcn_perm(js < 4 ? sh03 : sh47, js < 4 ? sh03 : sh47, sel);
            const uint32_t ml = __builtin_amdgcn_perm(js < 4 ? sl03 : sl47, js < 4 ? sl03 : sl47, sel);
            const v4i bh = v4i{ (int)mul_u16x2(n0, mh), (int)mul_u16x2(n1, mh), (int)mul_u16x2(n2, mh),
                                (int)mul_u16x2(n3, mh) };
            const v4i bl = v4i{ (int)mul_u16x2(n0, ml), (int)mul_u16x2(n1, ml), (int)mul_u16x2(n2, ml),
                                (int)mul_u16x2(n3, ml) };
            // (the last sub-block issues tile 0's two chains first: its combine below waits for
            // them only)
            acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bh, j ? acc[0] : v16i{}, 0, 0, 0);
            if (j == 7) acc[2] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bl, acc[2], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bh, j ? acc[1] : v16i{}, 0, 0, 0);
            if (j < 7) acc[2] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bl, j ? acc[2] : v16i{}, 0, 0, 0);
            acc[3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bl, j ? acc[3] : v16i{}, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        // min term sum_j m_j bsum_j of each column tile: A = the columns' split sums bh (then bl,
        // bsum = 64 bh + bl) at k = j, B = the row's 8 mins; the second MFMA starts from 64 * first
        // + the bits of 12582912.0f, so its result read as a float is 12582912 + imn exactly
        // (|imn| < 2^22).  Each tile's isc = 8 sum_sh + sum_sl (in place) runs under its first
        // min MFMA, and tile 1's min term under tile 0's second.
        float d = h2f(dd & 0xffffu), dmin = h2f(dd >> 16);
        asm volatile("" : "+v"(d), "+v"(dmin));               // f32 operands (no fp16 source folding)
        const float nmag = 12582912.0f * dmin;                // exact: fp16 dmin times 3 * 2^22
        const v4i bm = h ? v4i{} : v4i{ (int)mn03, (int)mn47, 0, 0 };
        v16i mlt[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint4 sp = *reinterpret_cast<const uint4 *>(S + 16384 + c * 512 + j32 * 16);
            const v4i ah = h ? v4i{} : v4i{ (int)sp.x, (int)sp.y, 0, 0 };
            const v4i al = h ? v4i{} : v4i{ (int)sp.z, (int)sp.w, 0, 0 };
            v16i mh = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, bm, v16i{}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[c][r] = (acc[c][r] << 3) + acc[2 + c][r];
#pragma unroll
            for (int r = 0; r < 16; ++r) mh[r] = mh[r] * 64 + kMagic;
            mlt[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, bm, mh, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        // the float combine of each column tile
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            float dx[16];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                // (output order: register r of half h is column 8 (r / 4) + 4 h + r % 4; the
                // grouped mode's scales lie in column order)
                const int off = GATHER ? 4 * (8 * q4 + 4 * h) : h * 64 + 16 * q4;
                const float4 v = *reinterpret_cast<const float4 *>(S + 17408 + c * 128 + off);
                dx[4 * q4] = v.x;
                dx[4 * q4 + 1] = v.y;
                dx[4 * q4 + 2] = v.z;
                dx[4 * q4 + 3] = v.w;
            }
            v16f & o = c ? out1 : out0;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                // (the element goes through a scalar: clang's __builtin_bit_cast of an ext-vector
                // element reads element 0)
                const int iml = mlt[c][r];
                const int isc = acc[c][r];
                const float wv = __builtin_fmaf(__builtin_bit_cast(float, iml), -dmin, nmag);   // -dmin * imn
                const float v = __builtin_fmaf((float)isc, d, wv);
                o[r] = __builtin_fmaf(v, dx[r], o[r]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // ---- K loop: super-block s + 1 goes into LDS while s is computed (its buffer was last read
    // before the previous barrier); the barrier's wait covers only these LDS loads, which are
    // issued before the iteration's weight loads
    stage(s0, 0);
#pragma unroll
    for (int c = 0; c < 4; ++c) ch[c] = bld16(wbuf, wl, (uint32_t)s0 * tgs + 2 * c * kChunk);
    hd = bld16(wbuf, row16, (uint32_t)s0 * tgs + 8 * kChunk);
    __syncthreads();
    for (int it = 0; it < p.sps; ++it) {                      // uniform over the work-group
        const int s = s0 + it;
        stage(std::min(s + 1, s1 - 1), (it + 1) & 1);         // (past the slice: a copy nobody reads)
        __builtin_amdgcn_sched_barrier(0);                    // the LDS loads go out before the weight loads
        if (s < s1) {
            compute(it & 1, s);
        } else {                                              // a slice shorter than sps: the same loads as
#pragma unroll                                                // compute's (unused), so that every path
            for (int c = 0; c < 4; ++c)                       // leaves them outstanding at the barrier
                ch[c] = bld16(wbuf, wl, (uint32_t)(s1 - 1) * tgs + 2 * c * kChunk);
            hd = bld16(wbuf, row16, (uint32_t)(s1 - 1) * tgs + 8 * kChunk);
        }
        // this wave's LDS loads are complete once at most the 5 weight loads issued after them
        // are outstanding (vmcnt(5)); the barrier then publishes them to the other waves
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(kVmcnt5);
        __syncthreads();
    }

    // ---- K slices 1.. add their sums into slice 0's through LDS (fixed order), slice 0 stores
    if (p.KS > 1) {
        float * red = reinterpret_cast<float *>(lds);
        if (ks > 0) {
            float * o = red + ((size_t)((ks - 1) * U + u) * 32) * 64 + lane;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                o[r * 64] = out0[r];
                o[(16 + r) * 64] = out1[r];
            }
        }
        __syncthreads();
        if (ks > 0) return;
        for (int k = 1; k < p.KS; ++k) {
            const float * o = red + ((size_t)((k - 1) * U + u) * 32) * 64 + lane;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                out0[r] += o[r * 64];
                out1[r] += o[(16 + r) * 64];
            }
        }
    }
    if (!row_ok) return;
    const int64_t m = mtile * kTileRows + 32 * t + j32;
    if (m >= p.w.M) return;
    if constexpr (GATHER) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const v16f & v = c ? out1 : out0;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int slot = 32 * c + 8 * (r >> 2) + 4 * h + (r & 3);
                if (slot < ncu) __builtin_nontemporal_store(v[r], p.dst + p.units[nb].dst_off[slot] + m);
            }
        }
        return;
    }
    float * dst = p.dst + (int64_t)i2 * p.bt.d_nb2 + (int64_t)i3 * p.bt.d_nb3 + m;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int64_t n0 = (2 * (int64_t)nb + c) * 32;
        const v16f & v = c ? out1 : out0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t n = n0 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (n < p.N) __builtin_nontemporal_store(v[r], dst + n * p.bt.d_nb1);
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

template <int U, bool GATHER>
hipError_t launch_kq(const KQParams & q, const G3Shape & sh, const dim3 & g, const dim3 & b, hipStream_t s,
                     const KTime * kt) {
    static const hipError_t attr = hipFuncSetAttribute((const void *)k_gemm3_q4k<U, GATHER>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    if (kt) hipExtLaunchKernelGGL(k_gemm3_q4k<U, GATHER>, g, b, (uint32_t)sh.lds, s, kt->start, kt->stop, 0, q);
    else k_gemm3_q4k<U, GATHER><<<g, b, sh.lds, s>>>(q);
    return hipGetLastError();
}

template <bool GATHER>
hipError_t launch_kq_u(const KQParams & q, const G3Shape & sh, const dim3 & g, const dim3 & b, hipStream_t s,
                       const KTime * kt) {
    switch (sh.U) {
        case 12: return launch_kq<12, GATHER>(q, sh, g, b, s, kt);
        case 6: return launch_kq<6, GATHER>(q, sh, g, b, s, kt);
        case 4: return launch_kq<4, GATHER>(q, sh, g, b, s, kt);
        case 3: return launch_kq<3, GATHER>(q, sh, g, b, s, kt);
        case 2: return launch_kq<2, GATHER>(q, sh, g, b, s, kt);
        default: return hipErrorInvalidValue;
    }
}

int env_int3(const char * name, int dflt) {
    const char * e = getenv(name);
    return e ? atoi(e) : dflt;
}

}  // namespace

bool gemm3_supported(int type) {
    if (env_int3("QMM_GEMM3", 1) == 0) return false;          // (read per call: tests switch them)
    return type == QMM_TYPE_Q4_0 || type == QMM_TYPE_Q8_0 || type == QMM_TYPE_IQ4_NL ||
           (type == QMM_TYPE_Q4_K && env_int3("QMM_GEMM3_Q4K", 1) != 0);
}

namespace {
// Q4_K launch shape: U row-half waves per K slice x KS slices, chosen by rounds of work-groups
// on the chip x super-blocks per slice: 12-wave work-groups fill a CU alone (3 waves per SIMD),
// whole rounds; 4-wave ones go three to a CU and a partial last round costs its fraction (the
// CUs take the next small group as one finishes; measured on 17408 x 5120 x 512: 4-wave groups
// 141 us, (6, 2) 145 us, (12, 1) 155 us).  Ties go to the earlier (larger U) candidate.
// ncp = column pairs (grouped mode: route units) per batch
bool kq_shape_ncp(const WView & w, int64_t ncp, int64_t nbatch, G3Shape * sh) {
    struct Cand { int U, KS, per_cu; };
    static const Cand cands[] = { { 12, 1, 1 }, { 6, 2, 1 }, { 4, 3, 1 }, { 3, 4, 1 }, { 4, 1, 3 }, { 2, 2, 3 } };
    const int64_t nrh = 2 * w.ntiles, G = w.G;
    const int cus = 256;
    int64_t best = -1;
    const int forced = env_int3("QMM_GEMM3_KQ", -1);           // index into cands (tuning)
    for (int i = 0; i < (int)(sizeof(cands) / sizeof(cands[0])); ++i) {
        if (forced >= 0 && i != forced) continue;
        const Cand & c = cands[i];
        const int64_t sps = (G + c.KS - 1) / c.KS, KS = (G + sps - 1) / sps;
        const int64_t mbn = (nrh + c.U - 1) / c.U, nwg = mbn * ncp * nbatch;
        const int64_t slots = (int64_t)cus * c.per_cu;
        // (in 1/64 rounds)
        const int64_t rounds = c.per_cu > 1 ? std::max<int64_t>(64, (nwg * 64 + slots - 1) / slots)
                                            : 64 * ((nwg + slots - 1) / slots);
        const int64_t cost = rounds * sps;
        if (best >= 0 && cost >= best) continue;
        best = cost;
        sh->U = c.U;
        sh->KS = (int)KS;
        sh->sps = (int)sps;
        sh->mbn = mbn;
    }
    if (best < 0) return false;
    sh->C = 2;
    sh->R = 32;
    sh->SB = 8;
    sh->nbn = ncp;
    sh->nst = (int)G;
    sh->threads = 64 * sh->U * sh->KS;
    sh->lds = std::max(sh->KS * 2 * kKQStage + (18 % sh->U ? 1024 : 0), (sh->KS - 1) * sh->U * 32 * 64 * 4);
    sh->workgroups = 8 * ((sh->mbn * ncp + 7) / 8) * nbatch;
    return sh->mbn * ncp < 0x7fffffff && sh->lds <= 160 * 1024 && sh->threads <= 64 * kKQMaxWaves;
}
bool kq_shape(const WView & w, int64_t N, int64_t nbatch, G3Shape * sh) {
    return kq_shape_ncp(w, ((N + 31) / 32 + 1) / 2, nbatch, sh);
}
}  // namespace

bool gemm3_id_supported(int type) { return type == QMM_TYPE_Q4_K && gemm3_supported(type); }

bool gemm3_id_shape(const WView & w, int64_t max_units, G3Shape * sh) {
    return gemm3_id_supported(QMM_TYPE_Q4_K) && max_units > 0 && w.G > 0 && w.ntiles > 0 &&
           kq_shape_ncp(w, max_units, 1, sh);
}

hipError_t launch_gemm3_id(int type, const WView & w, const ActBuf & a, const GemmUnit * units, const int32_t * nunits,
                           int64_t max_units, float * dst, hipStream_t s, const KTime * kt) {
    G3Shape sh;
    if (!gemm3_id_supported(type) || a.vdt != QMM_TYPE_Q8_K || !a.bsp || !units || !nunits || a.ldk != w.G * 256 ||
        !gemm3_id_shape(w, max_units, &sh) || a.ncols * a.ldk >= ((int64_t)1 << 31) ||
        w.G * a.ldT * 16 >= ((int64_t)1 << 31) || a.ldT < a.ncols)
        return hipErrorInvalidValue;
    KQParams q{};
    q.w = w;
    q.nsb = w.G;
    q.mbn = sh.mbn;
    q.nbn = max_units;
    q.total = sh.mbn * max_units;
    q.chunk = (q.total + 7) / 8;
    q.U = sh.U;
    q.KS = sh.KS;
    q.sps = sh.sps;
    q.bt = GemmBatch{ 1, 1, 1, 0, 0, 0, 0 };                 // (one batch: mat comes from the unit)
    q.dst = dst;
    q.units = units;
    q.nunits = nunits;
    q.codes = a.codes;
    q.dcol = a.d;
    q.bsp = a.bsp;
    q.ldk = a.ldk;
    q.ldT = a.ldT;
    q.ncols = a.ncols;
    const dim3 g((unsigned)(8 * q.chunk), 1u), b(sh.threads);
    return launch_kq_u<true>(q, sh, g, b, s, kt);
}

// Launch shape: C column tiles per wave (2 shares each weight unpack between two column tiles,
// at twice the accumulators), kU row tiles per work-group, and K slices so that the waves come
// to about `target` (3 per SIMD).
bool gemm3_shape(int type, const WView & w, int64_t N, int64_t nbatch, G3Shape * sh) {
    if (!gemm3_supported(type) || N <= 0 || nbatch <= 0 || nbatch > 65535 || w.G <= 0 || w.ntiles <= 0) return false;
    if (type == QMM_TYPE_Q4_K) return kq_shape(w, N, nbatch, sh);
    const int64_t ntb = (N + 31) / 32;
    sh->C = 1;
    sh->R = 64;
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
        a.ntiles != a.ntb * nbatch || a.vdt != vec_dot_type(type))
        return hipErrorInvalidValue;
    if (type == QMM_TYPE_Q4_K) {
        if (!a.S) return hipErrorInvalidValue;
        KQParams q{};
        q.w = w;
        q.tA = a.A;
        q.tD = a.D;
        q.tS = a.S;
        q.nsb = w.G;
        q.ntb = a.ntb;
        q.N = a.N;
        q.mbn = sh.mbn;
        q.nbn = sh.nbn;
        q.total = sh.mbn * sh.nbn;
        q.chunk = (q.total + 7) / 8;
        q.U = sh.U;
        q.KS = sh.KS;
        q.sps = sh.sps;
        q.bt = bt;
        q.dst = dst;
        const dim3 g((unsigned)(8 * q.chunk), (unsigned)nbatch), b(sh.threads);
        return launch_kq_u<false>(q, sh, g, b, s, kt);
    }
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
