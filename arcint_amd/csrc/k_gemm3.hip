// k_gemm3.hip - the streaming prefill GEMMs on gfx950 v_mfma_i32_32x32x32_i8: Q4_K
// (k_gemm3_q4k, also the grouped MoE GEMM) and the block types with one float scale per 32
// weights, Q4_0, Q8_0 and IQ4_NL (k_gemm3_blk), weights streamed by each wave.
//
// Role of the reference's int8 prefill GEMMs (kernel_mul_mm_kq2d_q4_0_i8, P0099:377-455;
// kernel_mul_mm_kq2d_q4_K_i8, P01:1919-2024) and its fp16 tile kernel for Q8_0
// (P02:4359-4384), redesigned for CDNA4 and for ggml-cpu's numerics.  Both kernels share one
// frame:
//  * a wave owns 32 rows (one half of a 64-row image tile) x 64 columns (two column tiles)
//    over one K slice and streams its rows' weights itself; lane (j, h) supplies row j's k
//    16 h .. 16 h + 15 of every 32 weights as the MFMA's B operand, and the output lane (j, h)
//    holds row j, so the lane's own row scales apply with no lane exchanges;
//  * the activations come from the pre-pass in MFMA A-operand order (1 KB per column tile and
//    32 weights) with their scales in MFMA output order; the U row-half waves of a K slice
//    (different rows, same columns) share a stage in LDS (256 weights of both column tiles,
//    18 KB), loaded by buffer loads that write LDS directly, one stage ahead, one barrier per
//    stage;
//  * three waves per SIMD (at most 168 registers): work-groups of 12 waves (U x KS) fill a CU
//    alone, 4-wave ones go three to a CU (shapes chosen by rounds of work-groups on the chip);
//  * the K slices of a row half are waves of one work-group: slices 1.. add their sums into LDS
//    at the end and slice 0 stores, so dst is written once (non-temporal), with no atomics and
//    no zeroing;
//  * every load goes through a buffer resource: the wave-uniform address math stays on the
//    SALU, and reads past a resource's range return zeros;
//  * work-groups that share weight rows are numbered onto one XCD (work-group b runs on XCD
//    b % 8), so a row tile's weights come from HBM once and from that XCD's L2 after.
// ggml's dot for the block types is sum_b d_x(b) d_w(b) I_b, a scale per 32-weight block on both
// sides, so every output takes a float multiply-add per block on top of the block's integer dot:
// two VALU instructions per output and block, 32 per MFMA, which bound that GEMM (the VALU, not
// the MFMA); Q4_K's scales fold into the int8 operands and its float combine runs once per 256.
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
// s_waitcnt immediates (gfx9 encoding): vmcnt 5 / 8 / 9 (bits 3:0, 15:14), expcnt and lgkmcnt not
// waited on
constexpr int kVmcnt5 = 5 | (0x7 << 4) | (0xF << 8);
constexpr int kVmcnt8 = 8 | (0x7 << 4) | (0xF << 8);
constexpr int kVmcnt9 = 9 | (0x7 << 4) | (0xF << 8);

struct KQParams {
    WView w;
    const int8_t * tA;
    const float * tD;
    const int8_t * tS;
    int64_t nsb;                         // super-blocks per column (the weights' groups)
    int64_t ntb;                         // column tiles per batch
    int64_t N;                           // columns per batch
    int64_t mbn, nbn;                    // work-group blocks per batch: U row halves along M, column pairs along N
    int64_t total;                       // mbn * nbn
    int U, KS, sps;                      // row-half waves per K slice, K slices, super-blocks per slice
    // blocks [0, full) whole, by 8 fchunk work-groups; the rest as ts pieces of pk super-blocks,
    // by 8 tchunk more, which meet in tree (tslots slots per output of a block's wave)
    int64_t full, fchunk, tchunk;
    int ts, pk, tslots;
    uint32_t * tree;
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
    // grouped mode with a GLU (glu >= 0): this launch is the up product, gsrc the gate product's
    // rows at the same offsets; stores act(gate) * up.  dspan: floats of dst (and gsrc) the
    // stores may reach, below 2^30
    const float * gsrc;
    int glu;
    int64_t dspan;
};

// The work-group's block L and K piece (-1: the whole K) from its index bx.  Blocks [0, full)
// come first, whole, XCD x (bx % 8) taking blocks x fchunk .. (x + 1) fchunk - 1, so the column
// pairs of one row block (neighbours in L) share their weight rows in one L2; then the tail's
// pieces e = ts (L - full) + i the same way.  false: no work (past the last block or piece).
__device__ __forceinline__ bool kq_block(const KQParams & p, uint32_t bx, uint32_t & L, int & piece) {
    const uint32_t fw = 8u * (uint32_t)p.fchunk;
    if (bx < fw) {
        L = (bx & 7) * (uint32_t)p.fchunk + (bx >> 3);
        piece = -1;
        return L < (uint32_t)p.full;
    }
    const uint32_t q = bx - fw, e = (q & 7) * (uint32_t)p.tchunk + (q >> 3);
    L = (uint32_t)p.full + e / (uint32_t)p.ts;
    piece = (int)(e % (uint32_t)p.ts);
    return e < (uint32_t)(p.total - p.full) * (uint32_t)p.ts;
}

// The ts pieces of a tail block add a wave's 32 sums per lane (out0, out1) up a pairwise tree of
// exchanges in slot memory, as the split GEMV's K slices do: at a level of n nodes, node i meets
// node i ^ 1 in slot i / 2 of the level (an odd last node moves up alone); the first arrival
// leaves its value and drops it, the second adds it to its own (a + b = b + a: the same sum
// whichever arrives first) and puts the slot back to kTreeEmpty.  Returns the mask of values
// this lane still holds at the root (to be stored); every slot ends empty.  nodes: the wave's
// slots, [slot][32 values][64 lanes].
__device__ __forceinline__ uint32_t kq_meet(uint32_t * nodes, int piece, int ts, v16f & out0, v16f & out1,
                                            int lane) {
    uint32_t live = 0xffffffffu;
    uint32_t i = (uint32_t)piece, n = (uint32_t)ts, off = 0;
    while (n > 1) {                                               // uniform
        if ((i ^ 1u) < n) {
            uint32_t * sl = nodes + (size_t)(off + (i >> 1)) * 2048 + lane;
            uint32_t o[32];
#pragma unroll
            for (int r = 0; r < 32; ++r) {
                const float v = r < 16 ? out0[r] : out1[r - 16];
                o[r] = (live >> r) & 1u ? __hip_atomic_exchange(sl + r * 64, __float_as_uint(v), __ATOMIC_RELAXED,
                                                                __HIP_MEMORY_SCOPE_AGENT)
                                        : kTreeEmpty;
            }
#pragma unroll
            for (int r = 0; r < 32; ++r) {
                if (!((live >> r) & 1u)) continue;
                if (o[r] == kTreeEmpty) {
                    live &= ~(1u << r);
                } else {
                    if (r < 16) out0[r] += __uint_as_float(o[r]);
                    else out1[r - 16] += __uint_as_float(o[r]);
                    __hip_atomic_store(sl + r * 64, kTreeEmpty, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        off += (n + 1) >> 1;
        i >>= 1;
        n = (n + 1) >> 1;
    }
    return live;
}

// v[i] = act(g[i]) * v[i] for one GLU op, as the split GLU computes it (glu_apply)
template <int OP>
__device__ __forceinline__ void glu_rows(const float (&g)[32], float (&v)[32]) {
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = glu_apply(OP, g[i], v[i]);
}

// the two 16-bit halves of v times those of s (v_pk_mul_lo_u16)
__device__ __forceinline__ uint32_t mul_u16x2(uint32_t v, uint32_t s) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, v) * __builtin_bit_cast(u16x2, s));
}

// a times s plus c in both 16-bit halves (v_pk_mad_u16: exact modulo 2^16, so signed too)
__device__ __forceinline__ uint32_t mad_u16x2(uint32_t a, uint32_t s, uint32_t c) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) * __builtin_bit_cast(u16x2, s) +
                                            __builtin_bit_cast(u16x2, c));
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

// Grouped mode's store of a wave's 32 sums per lane (rows m, the unit's 64 slots): each output
// goes to its pair's dst offset, read from the unit.  Every offset (and gate value) is requested
// before the first store, and no load or store sits in a branch: through buffer resources over
// dst's span an offset past it (kNoStore: a slot past the unit) reads zero and drops its store.
// (Conditional accesses, and loads after stores to dst that might alias them, made each of the 32
// stores wait for a memory round trip.)  With p.glu >= 0 the launch is the up product of a
// gate/up pair: act(gate) * up, gate read at the same offset.
__device__ __forceinline__ void gather_store(const KQParams & p, uint32_t nb, int ncu, int64_t m, int h,
                                             const v16f & out0, const v16f & out1) {
    constexpr uint32_t kNoStore = 0xffffffffu;
    const uint32_t span4 = (uint32_t)(p.dspan * 4);
    const __amdgpu_buffer_rsrc_t dres = buffer_rsrc(p.dst, span4);
    uint32_t off[32];
    float val[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int slot = 32 * (i >> 4) + 8 * ((i & 15) >> 2) + 4 * h + (i & 3);   // < 64: in the unit
        const int64_t o = p.units[nb].c[slot].dst_off + m;
        off[i] = slot < ncu ? 4u * (uint32_t)o : kNoStore;
        val[i] = i < 16 ? out0[i] : out1[i - 16];
    }
    if (p.glu >= 0) {                                         // uniform
        const __amdgpu_buffer_rsrc_t gres = buffer_rsrc(p.gsrc, span4);
        float gv[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) gv[i] = __uint_as_float(bld4(gres, off[i], 0));
        // one branch for the op, then straight-line code over the values
        switch (p.glu) {
            case QMM_GLU_REGLU: glu_rows<QMM_GLU_REGLU>(gv, val); break;
            case QMM_GLU_GEGLU: glu_rows<QMM_GLU_GEGLU>(gv, val); break;
            case QMM_GLU_SWIGLU: glu_rows<QMM_GLU_SWIGLU>(gv, val); break;
            case QMM_GLU_GEGLU_ERF: glu_rows<QMM_GLU_GEGLU_ERF>(gv, val); break;
            default: glu_rows<QMM_GLU_GEGLU_QUICK>(gv, val); break;
        }
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val[i]), dres, (int)off[i], 0, 0);
}

template <int U, bool GATHER>
__global__ __launch_bounds__(64 * kKQMaxWaves) void k_gemm3_q4k(KQParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, j32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int u = wave % U, ks = wave / U;

    uint32_t L;
    int piece;
    if (!kq_block(p, blockIdx.x, L, piece)) return;           // uniform over the work-group
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
    // the work-group's super-blocks [kb, ke): all, or its piece's
    const int kb = piece >= 0 ? piece * p.pk : 0, ke = piece >= 0 ? std::min(kb + p.pk, nsb) : nsb;
    const int sps = piece >= 0 ? p.pk : p.sps;                // (pieces: one K slice)
    const int s0 = kb + ks * sps;
    const int s1 = std::min(s0 + sps, ke);                    // (every slice has super-blocks)

    if (GATHER && mat < 0) {                                  // invalid ids: zero rows (uniform)
        const int64_t m = mtile * kTileRows + 32 * t + j32;
        if (!row_ok || m >= p.w.M || ks > 0) return;
        for (int n = h; n < ncu; n += 2) p.dst[p.units[nb].c[n].dst_off + m] = 0.0f;
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
            gcol[c] = slot < ncu ? (uint32_t)p.units[nb].c[slot].col : kOut;
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
                const uint32_t col = slot < ncu ? (uint32_t)p.units[nb].c[slot].col : kOut;
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
    for (int it = 0; it < sps; ++it) {                        // uniform over the work-group
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
        gather_store(p, nb, ncu, m, h, out0, out1);
        return;
    }
    // a tail piece: the block's pieces meet first, the holder of a sum stores it
    const uint32_t live = piece >= 0 ? kq_meet(p.tree + ((size_t)(L - p.full) * U + u) * (size_t)p.tslots * 2048, piece,
                                               p.ts, out0, out1, lane)
                                     : 0xffffffffu;
    float * dst = p.dst + (int64_t)i2 * p.bt.d_nb2 + (int64_t)i3 * p.bt.d_nb3 + m;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int64_t n0 = (2 * (int64_t)nb + c) * 32;
        const v16f & v = c ? out1 : out0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t n = n0 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (n < p.N && ((live >> (16 * c + r)) & 1u)) __builtin_nontemporal_store(v[r], dst + n * p.bt.d_nb1);
        }
    }
}

// ---- Q6_K ------------------------------------------------------------------------------------
// Role of the reference's Q6_K prefill GEMM (kernel_mul_mm_kq2d_q6_K, P01:1776-1860: fp16 DPAS on
// 1024 + code halves), on int8 MFMAs and ggml-cpu's numerics (q6_K x q8_K: an exact integer dot
// per 16-weight group times its int8 scale, summed per super-block, then d_w d_x).  The frame is
// k_gemm3_q4k's (32 rows x 64 columns per wave, q8_K activations staged in LDS one super-block
// ahead, weights streamed by each wave, K slices met in LDS, the tail in K pieces).
//  * The scaled weight p = sc (q - 32) takes 13 bits (in [-4064, 4096]), too many for an int8
//    operand.  Lane (j, h)'s 16 weights of sub-block s (32 weights) are exactly one scale group,
//    2 s + h, so each lane scales its own codes: two v_pk_mad_u16 per 4 codes give t = p + 128
//    in 16-bit lanes, and p = 256 H + L splits into two int8 operands, H = t >> 8 in [-16, 16]
//    (t's high bytes) and L = (int8) p (t's low bytes, bit 7 flipped), picked by v_perm.  Each
//    half has its own MFMA accumulator per column tile over the super-block: 4 MFMAs per
//    sub-block and wave, isum = 256 ah + al exact (ggml's per-group integer dots times the
//    scales).  (First written with the scale out of the operand: one MFMA per group on codes
//    masked to one lane half, then a v_mad_i32_i24 per output and group, ~870 VALU per
//    super-block against ~530.)
//  * Codes: weight k = 128 n + 32 s + l of the super-block is ql[64 n + 32 (s & 1) + l] (low
//    nibble for s < 2, high for s >= 2) with qh[32 n + l] bits 2 s, 2 s + 1 above it; lane half
//    h holds l in [16 h, 16 h + 16): ql chunk plane 4 n + 2 (s & 1) + h, qh plane 8 + 2 n + h.
//  * Per super-block and output: out += dx (d isum) (ggml's d_w d_x times the integer sum).
template <int U, bool GATHER>
__global__ __launch_bounds__(64 * kKQMaxWaves) void k_gemm3_q6k(KQParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, j32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int u = wave % U, ks = wave / U;

    uint32_t L;
    int piece;
    if (!kq_block(p, blockIdx.x, L, piece)) return;           // uniform over the work-group
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
    const int kb = piece >= 0 ? piece * p.pk : 0, ke = piece >= 0 ? std::min(kb + p.pk, nsb) : nsb;
    const int sps = piece >= 0 ? p.pk : p.sps;                // (pieces: one K slice)
    const int s0 = kb + ks * sps;
    const int s1 = std::min(s0 + sps, ke);                    // (every slice has super-blocks)

    if (GATHER && mat < 0) {                                  // invalid ids: zero rows (uniform)
        const int64_t m = mtile * kTileRows + 32 * t + j32;
        if (!row_ok || m >= p.w.M || ks > 0) return;
        for (int n = h; n < ncu; n += 2) p.dst[p.units[nb].c[n].dst_off + m] = 0.0f;
        return;
    }

    const __amdgpu_buffer_rsrc_t wbuf = buffer_rsrc(tile_group(p.w, mat, mtile, 0), (uint32_t)(p.w.G * p.w.tg));
    // (grouped mode: the route's whole quantization, each lane at its own column, as k_gemm3_q4k)
    const __amdgpu_buffer_rsrc_t abuf = GATHER ? buffer_rsrc(p.codes, (uint32_t)(p.ncols * p.ldk))
                                               : buffer_rsrc(p.tA + ct0 * p.nsb * 8192, (uint32_t)(nct * p.nsb * 8192));
    const __amdgpu_buffer_rsrc_t dbuf = GATHER ? buffer_rsrc(p.dcol, (uint32_t)(p.ncols * p.nsb * 4))
                                               : buffer_rsrc(p.tD + ct0 * p.nsb * 32, (uint32_t)(nct * p.nsb * 128));
    const uint32_t lane16 = (uint32_t)lane * 16;

    // ---- staging: k_gemm3_q4k's 18 units of 1 KB per super-block (A of both tiles; unit 16, the
    // split sums Q4_K takes, reads nothing here (an offset past the range: zeros into its slot) but
    // keeps every wave's load count; the scales)
    constexpr int NU = kq_units(U);
    constexpr uint32_t kOut = 0x7ff00000u;
    const uint32_t a_stride = (uint32_t)p.nsb * 8192, d_stride = (uint32_t)p.nsb * 128;
    uint32_t d_lane = lane < 16 ? (uint32_t)(lane >> 3) * d_stride + (uint32_t)(lane & 7) * 16 : kOut;
    // grouped mode (k_gemm3_q4k's layout): A unit (c, g) holds columns 4 g .. 4 g + 3 of tile c
    // whole, column i's 16-byte chunk q at LDS slot q ^ (i & 15); D by the lane's column
    uint32_t avo[NU];
#pragma unroll
    for (int k = 0; k < NU; ++k) avo[k] = 0;
    if constexpr (GATHER) {
        const int slot = 32 * (lane >> 5) + j32;
        const uint32_t gsd = slot < ncu ? (uint32_t)p.units[nb].c[slot].col : kOut;
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            const int unit = u + k * U;
            if (unit < 16) {
                const int ci = 4 * (unit & 7) + (lane >> 4);  // column of the tile
                const int cs = 32 * (unit >> 3) + ci;
                const uint32_t col = cs < ncu ? (uint32_t)p.units[nb].c[cs].col : kOut;
                const uint32_t q = (uint32_t)((lane & 15) ^ (ci & 15));
                avo[k] = col == kOut ? kOut : col * (uint32_t)p.ldk + 16 * q;
            }
        }
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
                dma16(dbuf, S + 16 * 1024, kOut, 0);
            } else if (unit == 17) {
                if (GATHER) dma4(dbuf, S + 17 * 1024, d_lane, (uint32_t)s * 4);   // [tile][32] f32 in column order
                else dma16(dbuf, S + 17 * 1024, d_lane, (uint32_t)s * 128);
            } else {
                dma16(dbuf, dump, kOut, 0);                   // (nothing: keeps the count)
            }
        }
    };

    // ---- weights of the lane's row (32 t + j32): ql planes 4 n + 2 c + h (c = s & 1), qh planes
    // 8 + 2 n + h, the 16 scales (plane 12), d (the tail's 2 bytes, in the row pair's dword)
    const uint32_t row = (uint32_t)(32 * t + j32), row16 = row * 16;
    const uint32_t tgs = (uint32_t)p.w.tg;
    auto plane = [&](int pl) { return row16 + (uint32_t)(pl + h) * kChunk; };   // (pl: the h = 0 plane)
    const uint32_t d_off = 13u * kChunk + (row & ~1u) * 2;
    uint4 ql[4], qh[2], sc;                                   // ql[2 n + c]
    uint32_t dw;
    auto wload = [&](uint32_t sb) {
#pragma unroll
        for (int n = 0; n < 2; ++n) {
#pragma unroll
            for (int c = 0; c < 2; ++c) ql[2 * n + c] = bld16(wbuf, plane(4 * n + 2 * c), sb);
            qh[n] = bld16(wbuf, plane(8 + 2 * n), sb);
        }
        sc = bld16(wbuf, row16 + 12 * kChunk, sb);
        dw = bld4(wbuf, d_off, sb);
    };

    v16f out0 = v16f{}, out1 = v16f{};                       // column tiles 0 and 1 of the pair
    auto compute = [&](int b, int s) {
        const uint8_t * S = lds + (ks * 2 + b) * kKQStage;
        // each plane is reloaded with the next super-block's as soon as its last sub-block has
        // used it (8 loads in all: the barrier's wait counts them)
        const uint32_t sn = (uint32_t)std::min(s + 1, s1 - 1) * tgs;
        const uint32_t cdw = dw;
        // lane (j32, h) holds group 2 j + h of sub-block j: its 16 products p = sc (q - 32) (13
        // bits signed, in [-4064, 4096]) come from two packed 16-bit multiply-adds per dword, as
        // t = p + 128, and split as p = 256 H + L: L = (int8) p, the low byte of t with bit 7
        // flipped, and H = t >> 8 in [-16, 16], t's high byte: two int8 operands, each MFMA
        // adding into its accumulator over the super-block (isum = 256 ah + al, exact)
        v16i ah0, ah1, al0, al1;
        // the A operands of sub-block j of both column tiles (grouped mode: chunk 2 j + h of column
        // j32 at its swizzled slot), read one sub-block ahead
        auto aread = [&](int j, v4i & x0, v4i & x1) {
            const uint32_t aoff = GATHER ? (uint32_t)j32 * 256 + 16 * (uint32_t)((2 * j + h) ^ (j32 & 15))
                                         : (uint32_t)(j * 1024) + lane16;
            x0 = *reinterpret_cast<const v4i *>(S + aoff);
            x1 = *reinterpret_cast<const v4i *>(S + 8192 + aoff);
        };
        v4i na0, na1;
        aread(0, na0, na1);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int n = j >> 2, sj = j & 3;
            const uint4 q = ql[2 * n + (sj & 1)], hb = qh[n];
            // the lane's group scale (byte 2 j + h of plane 12) and 128 - 32 sc, in both 16-bit halves
            const uint32_t sw = (j >> 1) == 0 ? sc.x : (j >> 1) == 1 ? sc.y : (j >> 1) == 2 ? sc.z : sc.w;
            const int sg = __builtin_amdgcn_sbfe((int)sw, 16 * (j & 1) + 8 * h, 8);
            const uint32_t s2 = __builtin_amdgcn_perm((uint32_t)sg, (uint32_t)sg, 0x01000100u);
            const uint32_t c2 = mad_u16x2(s2, 0xffe0ffe0u, 0x00800080u);   // 128 - 32 sc
            auto split = [&](uint32_t lo, uint32_t hi, int & bh, int & bl) {
                const uint32_t nib = (sj < 2 ? lo : lo >> 4) & 0x0F0F0F0Fu;
                const uint32_t hs = sj == 0 ? hi << 4 : sj == 1 ? hi << 2 : sj == 2 ? hi : hi >> 2;
                // codes 0..63, bytes 0..3 = weights 0..3: (hs & 0x30303030) | nib in one v_bitop3
                const uint32_t qv = __builtin_amdgcn_bitop3_b32(hs, 0x30303030u, nib, 0xEA);
                const uint32_t te = mad_u16x2(qv & 0x00ff00ffu, s2, c2);                          // weights 0, 2
                const uint32_t to = mad_u16x2(__builtin_amdgcn_perm(qv, qv, 0x0c030c01u), s2, c2);   // weights 1, 3
                // (bytes of the 16-bit lanes back in weight order: te, to, te, to)
                bh = (int)__builtin_amdgcn_perm(to, te, 0x07030501u);
                bl = (int)(__builtin_amdgcn_perm(to, te, 0x06020400u) ^ 0x80808080u);
            };
            int h0, h1, h2, h3, l0, l1, l2, l3;
            split(q.x, hb.x, h0, l0);
            split(q.y, hb.y, h1, l1);
            split(q.z, hb.z, h2, l2);
            split(q.w, hb.w, h3, l3);
            const v4i bh = v4i{ h0, h1, h2, h3 }, bl = v4i{ l0, l1, l2, l3 };
            const v4i a0 = na0, a1 = na1;
            if (j < 7) aread(j + 1, na0, na1);
            if (sj >= 2) ql[2 * n + (sj & 1)] = bld16(wbuf, plane(4 * n + 2 * (sj & 1)), sn);   // (its last use)
            if (sj == 3) qh[n] = bld16(wbuf, plane(8 + 2 * n), sn);
            if (j == 7) {
                sc = bld16(wbuf, row16 + 12 * kChunk, sn);
                dw = bld4(wbuf, d_off, sn);
            }
            ah0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bh, j ? ah0 : v16i{}, 0, 0, 0);
            ah1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bh, j ? ah1 : v16i{}, 0, 0, 0);
            al0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bl, j ? al0 : v16i{}, 0, 0, 0);
            al1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bl, j ? al1 : v16i{}, 0, 0, 0);
        }
        // the float combine of each column tile: out += dx (d isum)
        float d = h2f(cdw >> (16 * (row & 1)));
        asm volatile("" : "+v"(d));                           // f32 operand (no fp16 source folding)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            float dx[16];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                // (output order; grouped mode: the scales lie in column order)
                const int off = GATHER ? 4 * (8 * q4 + 4 * h) : h * 64 + 16 * q4;
                const float4 v = *reinterpret_cast<const float4 *>(S + 17408 + c * 128 + off);
                dx[4 * q4] = v.x;
                dx[4 * q4 + 1] = v.y;
                dx[4 * q4 + 2] = v.z;
                dx[4 * q4 + 3] = v.w;
            }
            v16f & o = c ? out1 : out0;
            const v16i & ah = c ? ah1 : ah0;
            const v16i & al = c ? al1 : al0;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int iv = ah[r] * 256 + al[r];
                o[r] = __builtin_fmaf((float)iv * d, dx[r], o[r]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // ---- K loop (k_gemm3_q4k's): super-block s + 1 goes into LDS while s is computed; the
    // barrier's wait covers only these LDS loads, issued before the iteration's 8 weight loads
    stage(s0, 0);
    wload((uint32_t)s0 * tgs);
    __syncthreads();
    for (int it = 0; it < sps; ++it) {                        // uniform over the work-group
        const int s = s0 + it;
        stage(std::min(s + 1, s1 - 1), (it + 1) & 1);         // (past the slice: a copy nobody reads)
        __builtin_amdgcn_sched_barrier(0);
        if (s < s1) compute(it & 1, s);
        else wload((uint32_t)(s1 - 1) * tgs);                 // (the same loads, unused: the wait below counts them)
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(kVmcnt8);
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
        gather_store(p, nb, ncu, m, h, out0, out1);
        return;
    }
    const uint32_t live = piece >= 0 ? kq_meet(p.tree + ((size_t)(L - p.full) * U + u) * (size_t)p.tslots * 2048, piece,
                                               p.ts, out0, out1, lane)
                                     : 0xffffffffu;
    float * dst = p.dst + (int64_t)i2 * p.bt.d_nb2 + (int64_t)i3 * p.bt.d_nb3 + m;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int64_t n0 = (2 * (int64_t)nb + c) * 32;
        const v16f & v = c ? out1 : out0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t n = n0 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (n < p.N && ((live >> (16 * c + r)) & 1u)) __builtin_nontemporal_store(v[r], dst + n * p.bt.d_nb1);
        }
    }
}

// ---- IQ4_XS and Q5_K: one integer scale per 32-weight sub-block ----------------------------
// Role of the reference's Q5_K and IQ4_XS prefill GEMMs (kernel_mul_mm_kq2d_q5_K, P01:1734-1775;
// kernel_mul_mm_iq4_xs_f16 over deq_iq4_xs, P01:2288-2310 and P01:2505-2507), on int8 MFMAs and
// ggml-cpu's numerics (an exact integer dot per sub-block times its integer scale; Q5_K's min
// term per super-block), on k_gemm3_q6k's frame.
//  * A sub-block's 32 weights share one scale (IQ4_XS: ls - 32, ls the 6-bit scale; Q5_K: the
//    6-bit sc), whose product with a code does not fit an int8 operand.  Both lane halves carry
//    sub-block j (lane (j, h): k 16 h .. 16 h + 15), so one MFMA per column tile gives its integer
//    dot for 32 x 32 outputs and a v_mad_i32_i24 per output adds it times the row's scale: 2 MFMAs
//    and 32 multiply-adds per sub-block and wave.
//  * IQ4_XS: chunk plane j holds sub-block j's 16 code bytes (low nibbles k 0..15, high 16..31),
//    lane h takes nibble h through the codebook; the tail's 8 bytes per row: d, scales_h,
//    scales_l[4] (ls = scales_l nibble j | scales_h bits 2 j, 2 j + 1 above it).
//  * Q5_K: Q4_K's planes (2 c + h: sub-blocks 2 c, 2 c + 1 in the nibbles) and header, the qh
//    planes 9 + h (bit j of byte l: the fifth bit of weight l of sub-block j); codes 0..31; the
//    min term as k_gemm3_q4k's (two MFMAs per column tile over the split sums and the mins).
//  * Per super-block and output: out += dx (d isum) (IQ4_XS), dx (d isum - dmin imn) (Q5_K).
template <int TYPE, int U, bool GATHER>
__global__ __launch_bounds__(64 * kKQMaxWaves) void k_gemm3_sbs(KQParams p) {
    constexpr bool Q5 = TYPE == QMM_TYPE_Q5_K;
    constexpr int kVm = Q5 ? (6 | (0x7 << 4) | (0xF << 8)) : (10 | (0x7 << 4) | (0xF << 8));   // weight loads a super-block
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, j32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int u = wave % U, ks = wave / U;

    uint32_t L;
    int piece;
    if (!kq_block(p, blockIdx.x, L, piece)) return;           // uniform over the work-group
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
    const int kb = piece >= 0 ? piece * p.pk : 0, ke = piece >= 0 ? std::min(kb + p.pk, nsb) : nsb;
    const int sps = piece >= 0 ? p.pk : p.sps;                // (pieces: one K slice)
    const int s0 = kb + ks * sps;
    const int s1 = std::min(s0 + sps, ke);                    // (every slice has super-blocks)

    if (GATHER && mat < 0) {                                  // invalid ids: zero rows (uniform)
        const int64_t m = mtile * kTileRows + 32 * t + j32;
        if (!row_ok || m >= p.w.M || ks > 0) return;
        for (int n = h; n < ncu; n += 2) p.dst[p.units[nb].c[n].dst_off + m] = 0.0f;
        return;
    }

    const __amdgpu_buffer_rsrc_t wbuf = buffer_rsrc(tile_group(p.w, mat, mtile, 0), (uint32_t)(p.w.G * p.w.tg));
    // (grouped mode: the route's whole quantization, each lane at its own column, as k_gemm3_q4k)
    const __amdgpu_buffer_rsrc_t abuf = GATHER ? buffer_rsrc(p.codes, (uint32_t)(p.ncols * p.ldk))
                                               : buffer_rsrc(p.tA + ct0 * p.nsb * 8192, (uint32_t)(nct * p.nsb * 8192));
    const __amdgpu_buffer_rsrc_t sbuf = GATHER ? buffer_rsrc(p.bsp, (uint32_t)(p.nsb * p.ldT * 16))
                                               : buffer_rsrc(p.tS + ct0 * p.nsb * 512, (uint32_t)(nct * p.nsb * 512));
    const __amdgpu_buffer_rsrc_t dbuf = GATHER ? buffer_rsrc(p.dcol, (uint32_t)(p.ncols * p.nsb * 4))
                                               : buffer_rsrc(p.tD + ct0 * p.nsb * 32, (uint32_t)(nct * p.nsb * 128));
    const uint32_t lane16 = (uint32_t)lane * 16;

    // ---- staging: k_gemm3_q4k's 18 units of 1 KB per super-block (the split sums read by Q5_K's
    // min term; IQ4_XS reads nothing into their slot but keeps every wave's load count)
    constexpr int NU = kq_units(U);
    constexpr uint32_t kOut = 0x7ff00000u;
    const uint32_t a_stride = (uint32_t)p.nsb * 8192, s_stride = (uint32_t)p.nsb * 512, d_stride = (uint32_t)p.nsb * 128;
    uint32_t s_lane = Q5 ? (uint32_t)(lane >> 5) * s_stride + (uint32_t)j32 * 16 : kOut;
    uint32_t d_lane = lane < 16 ? (uint32_t)(lane >> 3) * d_stride + (uint32_t)(lane & 7) * 16 : kOut;
    // grouped mode (k_gemm3_q4k's layout): A unit (c, g) holds columns 4 g .. 4 g + 3 of tile c
    // whole, column i's 16-byte chunk q at LDS slot q ^ (i & 15); S and D by the lane's column
    uint32_t avo[NU];
#pragma unroll
    for (int k = 0; k < NU; ++k) avo[k] = 0;
    if constexpr (GATHER) {
        uint32_t gcol[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int slot = 32 * c + j32;
            gcol[c] = slot < ncu ? (uint32_t)p.units[nb].c[slot].col : kOut;
        }
        const uint32_t gsd = (lane >> 5) ? gcol[1] : gcol[0];
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            const int unit = u + k * U;
            if (unit < 16) {
                const int ci = 4 * (unit & 7) + (lane >> 4);  // column of the tile
                const int slot = 32 * (unit >> 3) + ci;
                const uint32_t col = slot < ncu ? (uint32_t)p.units[nb].c[slot].col : kOut;
                const uint32_t q = (uint32_t)((lane & 15) ^ (ci & 15));
                avo[k] = col == kOut ? kOut : col * (uint32_t)p.ldk + 16 * q;
            }
        }
        s_lane = Q5 && gsd != kOut ? gsd * 16 : kOut;
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
                dma16(Q5 ? sbuf : dbuf, S + 16 * 1024, s_lane,
                      !Q5 ? 0u : GATHER ? (uint32_t)(s * p.ldT * 16) : (uint32_t)s * 512);
            } else if (unit == 17) {
                if (GATHER) dma4(dbuf, S + 17 * 1024, d_lane, (uint32_t)s * 4);   // [tile][32] f32 in column order
                else dma16(dbuf, S + 17 * 1024, d_lane, (uint32_t)s * 128);
            } else {
                dma16(dbuf, dump, kOut, 0);                   // (nothing: keeps the count)
            }
        }
    };

    // ---- weights of the lane's row (32 t + j32)
    const uint32_t row = (uint32_t)(32 * t + j32), row16 = row * 16;
    const uint32_t tgs = (uint32_t)p.w.tg;
    // IQ4_XS: planes j (8), the tail's two dwords; Q5_K: planes 2 c + h (4), the header, qh plane 9 + h
    constexpr int NP = Q5 ? 4 : 8;
    uint4 pl[NP], hd;                                         // (hd: Q5_K's header, IQ4_XS's tail in .x, .y)
    uint4 qh = uint4{ 0, 0, 0, 0 };
    auto pl_off = [&](int c) { return Q5 ? row16 + (uint32_t)(2 * c + h) * kChunk : row16 + (uint32_t)c * kChunk; };
    const uint32_t tail = 8u * kChunk + row * 8;
    auto hload = [&](uint32_t sb) {
        if constexpr (Q5) {
            hd = bld16(wbuf, row16 + 8 * kChunk, sb);
            qh = bld16(wbuf, row16 + (uint32_t)(9 + h) * kChunk, sb);
        } else {
            hd.x = bld4(wbuf, tail, sb);
            hd.y = bld4(wbuf, tail + 4, sb);
        }
    };
    const uint32_t nsh = 4u * (uint32_t)h;                    // IQ4_XS: the lane half's nibble

    v16f out0 = v16f{}, out1 = v16f{};                       // column tiles 0 and 1 of the pair
    auto compute = [&](int b, int s) {
        const uint8_t * S = lds + (ks * 2 + b) * kKQStage;
        const uint32_t sn = (uint32_t)std::min(s + 1, s1 - 1) * tgs;   // the next super-block (clamped)
        // the row's scales (and Q5_K's mins and fifth bits) from this super-block's header, whose
        // registers are reloaded with the next one's at once
        const uint4 chd = hd, cqh = qh;
        hload(sn);
        uint32_t sc03, sc47, mn03 = 0, mn47 = 0;
        if constexpr (Q5) {
            sc03 = chd.y & 0x3f3f3f3fu;
            mn03 = chd.z & 0x3f3f3f3fu;
            sc47 = (chd.w & 0x0f0f0f0fu) | ((chd.y >> 2) & 0x30303030u);
            mn47 = ((chd.w >> 4) & 0x0f0f0f0fu) | ((chd.z >> 2) & 0x30303030u);
        } else {
            sc03 = chd.y;                                     // scales_l (nibble j = bits 4 j)
            sc47 = chd.x >> 16;                               // scales_h (bits 2 j, 2 j + 1)
        }
        v16i is0 = v16i{}, is1 = v16i{};                      // the super-block's integer sums
        // the A operands of sub-block j of both column tiles (grouped mode: chunk 2 j + h of column
        // j32 at its swizzled slot), read one sub-block ahead
        auto aread = [&](int j, v4i & x0, v4i & x1) {
            const uint32_t aoff = GATHER ? (uint32_t)j32 * 256 + 16 * (uint32_t)((2 * j + h) ^ (j32 & 15))
                                         : (uint32_t)(j * 1024) + lane16;
            x0 = *reinterpret_cast<const v4i *>(S + aoff);
            x1 = *reinterpret_cast<const v4i *>(S + 8192 + aoff);
        };
        v4i na0, na1;
        aread(0, na0, na1);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v4i bop;
            if constexpr (Q5) {
                const uint4 q = pl[j >> 1];
                const uint32_t ns = 4u * (uint32_t)(j & 1);
                auto code = [&](uint32_t w, uint32_t hb) {
                    const uint32_t fifth = (j <= 4 ? hb << (4 - j) : hb >> (j - 4)) & 0x10101010u;
                    return ((w >> ns) & 0x0F0F0F0Fu) | fifth;
                };
                bop = v4i{ (int)code(q.x, cqh.x), (int)code(q.y, cqh.y), (int)code(q.z, cqh.z), (int)code(q.w, cqh.w) };
                if (j & 1) pl[j >> 1] = bld16(wbuf, pl_off(j >> 1), sn);   // (its last sub-block)
            } else {
                const uint4 q = pl[j];
                bop = v4i{ (int)iq4_lookup((q.x >> nsh) & 0x0F0F0F0Fu), (int)iq4_lookup((q.y >> nsh) & 0x0F0F0F0Fu),
                           (int)iq4_lookup((q.z >> nsh) & 0x0F0F0F0Fu), (int)iq4_lookup((q.w >> nsh) & 0x0F0F0F0Fu) };
                pl[j] = bld16(wbuf, pl_off(j), sn);
            }
            const v4i a0 = na0, a1 = na1;
            if (j < 7) aread(j + 1, na0, na1);
            int sc;
            if constexpr (Q5) {
                sc = (int)__builtin_amdgcn_ubfe(j < 4 ? sc03 : sc47, 8 * (j & 3), 8);
            } else {
                sc = (int)(__builtin_amdgcn_ubfe(sc03, 4 * j, 4) | (__builtin_amdgcn_ubfe(sc47, 2 * j, 2) << 4)) - 32;
            }
            const v16i p0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bop, v16i{}, 0, 0, 0);
            const v16i p1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bop, v16i{}, 0, 0, 0);
            // (the sums are made opaque after each sub-block: the compiler would otherwise
            // reassociate them across the sub-blocks and keep every MFMA result)
#pragma unroll
            for (int r = 0; r < 16; ++r) is0[r] = __mul24(sc, p0[r]) + is0[r];
#pragma unroll
            for (int r = 0; r < 16; ++r) is1[r] = __mul24(sc, p1[r]) + is1[r];
            asm volatile("" : "+v"(is0), "+v"(is1));
            __builtin_amdgcn_sched_barrier(0);
        }
        // the float combine of each column tile
        float d, dmin = 0.0f;
        if constexpr (Q5) {
            d = h2f(chd.x & 0xffffu);
            dmin = h2f(chd.x >> 16);
        } else {
            d = h2f(chd.x & 0xffffu);
        }
        asm volatile("" : "+v"(d), "+v"(dmin));               // f32 operands (no fp16 source folding)
        v16i mlt[2];
        if constexpr (Q5) {
            // Q5_K's min term (k_gemm3_q4k's): A = the columns' split sums bh, then bl, at k = j, B
            // = the row's 8 mins; the second MFMA starts from 64 * first + the bits of 12582912.0f
            const v4i bm = h ? v4i{} : v4i{ (int)mn03, (int)mn47, 0, 0 };
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const uint4 sp = *reinterpret_cast<const uint4 *>(S + 16384 + c * 512 + j32 * 16);
                const v4i ah = h ? v4i{} : v4i{ (int)sp.x, (int)sp.y, 0, 0 };
                const v4i al = h ? v4i{} : v4i{ (int)sp.z, (int)sp.w, 0, 0 };
                v16i mh = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, bm, v16i{}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; ++r) mh[r] = mh[r] * 64 + kMagic;
                mlt[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, bm, mh, 0, 0, 0);
            }
        }
        const float nmag = 12582912.0f * dmin;                // exact: fp16 dmin times 3 * 2^22
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            float dx[16];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                // (output order; grouped mode: the scales lie in column order)
                const int off = GATHER ? 4 * (8 * q4 + 4 * h) : h * 64 + 16 * q4;
                const float4 v = *reinterpret_cast<const float4 *>(S + 17408 + c * 128 + off);
                dx[4 * q4] = v.x;
                dx[4 * q4 + 1] = v.y;
                dx[4 * q4 + 2] = v.z;
                dx[4 * q4 + 3] = v.w;
            }
            v16f & o = c ? out1 : out0;
            const v16i & is = c ? is1 : is0;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int iv = is[r];
                if constexpr (Q5) {
                    const int iml = mlt[c][r];
                    const float wv = __builtin_fmaf(__builtin_bit_cast(float, iml), -dmin, nmag);   // -dmin * imn
                    o[r] = __builtin_fmaf(__builtin_fmaf((float)iv, d, wv), dx[r], o[r]);
                } else {
                    o[r] = __builtin_fmaf((float)iv * d, dx[r], o[r]);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // ---- K loop (k_gemm3_q4k's): super-block s + 1 goes into LDS while s is computed; the
    // barrier's wait covers only these LDS loads, issued before the iteration's weight loads
    auto wload_all = [&](uint32_t sb) {
#pragma unroll
        for (int c = 0; c < NP; ++c) pl[c] = bld16(wbuf, pl_off(c), sb);
        hload(sb);
    };
    stage(s0, 0);
    wload_all((uint32_t)s0 * tgs);
    __syncthreads();
    for (int it = 0; it < sps; ++it) {                        // uniform over the work-group
        const int s = s0 + it;
        stage(std::min(s + 1, s1 - 1), (it + 1) & 1);         // (past the slice: a copy nobody reads)
        __builtin_amdgcn_sched_barrier(0);
        if (s < s1) compute(it & 1, s);
        else wload_all((uint32_t)(s1 - 1) * tgs);             // (the same loads, unused: the wait below counts them)
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(kVm);
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
        gather_store(p, nb, ncu, m, h, out0, out1);
        return;
    }
    const uint32_t live = piece >= 0 ? kq_meet(p.tree + ((size_t)(L - p.full) * U + u) * (size_t)p.tslots * 2048, piece,
                                               p.ts, out0, out1, lane)
                                     : 0xffffffffu;
    float * dst = p.dst + (int64_t)i2 * p.bt.d_nb2 + (int64_t)i3 * p.bt.d_nb3 + m;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int64_t n0 = (2 * (int64_t)nb + c) * 32;
        const v16f & v = c ? out1 : out0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t n = n0 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (n < p.N && ((live >> (16 * c + r)) & 1u)) __builtin_nontemporal_store(v[r], dst + n * p.bt.d_nb1);
        }
    }
}

// ---- Q4_0, Q8_0, IQ4_NL: the streaming form with 32-row x 64-column waves -----------------
// The block types on the Q4_K kernel's frame: a wave owns 32 rows (one half of a 64-row image
// tile) x 64 columns (two column tiles) over one K slice, the U row-half waves of a K slice
// share a stage of activations in LDS (one 256-weight group: both tiles' A operands, 16 KB, and
// their f32 scales, 2 KB, by buffer loads that write LDS directly), one barrier per group.
//  * lane (j, h) supplies row j's k 16 h .. 16 h + 15 of every block as the MFMA's B operand,
//    and the output lane (j, h) holds row j: the lane's own row scale d_w applies, no lane
//    exchanges.  Q4_0 / IQ4_NL: the lane loads the row's 16 bytes of the block and takes the low
//    (h = 0) or high (h = 1) nibbles; Q8_0: the lane loads the row's code plane h of the block;
//  * one weight unpack feeds the MFMAs of both column tiles (the 64 x 32 form unpacks once per
//    column tile and trades lane halves with v_permlane32_swap): ~75 VALU per 2 MFMAs, against
//    ~91, of which 64 are ggml's float combine (two FMAs per output and block);
//  * Q4_0 codes enter as (q ^ 8) << 4 = 16 (q - 8) (no borrow handling), the sums carrying the
//    factor 16 taken off exactly at the store;
//  * the MFMA's C input is the bits of 12582912.0f: its result read as a float is 12582912 + I
//    exactly, fma(that, d_w, -12582912 d_w) is I d_w rounded once and fma(., d_x, acc)
//    accumulates it (ggml's per-block combine);
//  * the lane's weights stream one group ahead: a block's chunk is reloaded with the next
//    group's as soon as its MFMAs are issued.
template <int TYPE, int U>
__global__ __launch_bounds__(64 * kKQMaxWaves) void k_gemm3_blk(KQParams p) {
    constexpr bool Q8 = TYPE == QMM_TYPE_Q8_0;
    constexpr bool NLQ = TYPE == QMM_TYPE_IQ4_NL;
    constexpr int kDch = Q8 ? 16 : 8;                         // chunk plane of the block scales
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, j32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int u = wave % U, ks = wave / U;

    uint32_t L;
    int piece;
    if (!kq_block(p, blockIdx.x, L, piece)) return;           // uniform over the work-group
    const uint32_t mb = L / (uint32_t)p.nbn, nb = L - mb * (uint32_t)p.nbn;
    const uint32_t bz = blockIdx.y;
    const uint32_t i2 = bz % (uint32_t)p.bt.ne12, i3 = bz / (uint32_t)p.bt.ne12;
    const int64_t mat = (int64_t)(i2 / (uint32_t)p.bt.r2) + (int64_t)(i3 / (uint32_t)p.bt.r3) * p.bt.ne02;
    const int64_t rh_raw = (int64_t)mb * U + u;               // the wave's row half
    const bool row_ok = rh_raw < 2 * p.w.ntiles;              // a missing row half computes a copy, stores nothing
    const int64_t rh = row_ok ? rh_raw : 2 * p.w.ntiles - 1;
    const int64_t mtile = rh >> 1;
    const int t = (int)(rh & 1);
    const int64_t ct0 = (int64_t)bz * p.ntb + 2 * (int64_t)nb; // the pair's first column tile
    const int64_t nct = std::min<int64_t>(2, p.ntb - 2 * (int64_t)nb);
    const int ng = (int)p.nsb;                                // groups (256 weights) along K
    // the work-group's groups [kb, ke): all, or its piece's
    const int kb = piece >= 0 ? piece * p.pk : 0, ke = piece >= 0 ? std::min(kb + p.pk, ng) : ng;
    const int sps = piece >= 0 ? p.pk : p.sps;                // (pieces: one K slice)
    const int s0 = kb + ks * sps;
    const int s1 = std::min(s0 + sps, ke);                    // (every slice has groups)
    const int64_t nblk = 8 * p.nsb;                           // blocks per activation column

    const __amdgpu_buffer_rsrc_t wbuf = buffer_rsrc(tile_group(p.w, mat, mtile, 0), (uint32_t)(p.w.G * p.w.tg));
    // the pair's activations; a pair with one tile reads zeros for the second (past the range)
    const __amdgpu_buffer_rsrc_t abuf = buffer_rsrc(p.tA + ct0 * nblk * 1024, (uint32_t)(nct * nblk * 1024));
    const __amdgpu_buffer_rsrc_t dbuf = buffer_rsrc(p.tD + ct0 * nblk * 32, (uint32_t)(nct * nblk * 128));
    const uint32_t lane16 = (uint32_t)lane * 16;

    // ---- staging of group s into buffer b of the slice: 18 units of 1 KB (A: tile unit / 8,
    // block unit % 8; the scales of tile unit - 16), wave u taking units u, u + U, ...
    constexpr int NU = kq_units(U);
    constexpr uint32_t kOut = 0x7ff00000u;
    const uint32_t a_stride = (uint32_t)(nblk * 1024), d_stride = (uint32_t)(nblk * 128);
    uint8_t * const dump = lds + 2 * p.KS * kKQStage;
    auto stage = [&](int s, int b) {
        uint8_t * S = lds + (ks * 2 + b) * kKQStage;
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            const int unit = u + i * U;                       // wave-uniform
            if (unit < 16)
                dma16(abuf, S + unit * 1024, lane16 + (uint32_t)(unit >> 3) * a_stride + (uint32_t)(unit & 7) * 1024,
                      (uint32_t)s * 8192);
            else if (unit < 18)
                dma16(dbuf, S + unit * 1024, lane16 + (uint32_t)(unit - 16) * d_stride, (uint32_t)s * 1024);
            else
                dma16(dbuf, dump, kOut, 0);                   // (nothing: keeps the count)
        }
    };

    // ---- weights of the lane's row (32 t + j32): per block the row's 16 bytes (Q8_0: its code
    // plane h), and the row's 8 block scales
    const uint32_t row16 = (uint32_t)(32 * t + j32) * 16;
    const uint32_t tgs = (uint32_t)p.w.tg;
    auto wplane = [&](int jb) -> uint32_t { return (uint32_t)(Q8 ? 2 * jb + h : jb) * kChunk; };
    uint4 wq[8], wd;

    v16f out0 = v16f{}, out1 = v16f{};                       // column tiles 0 and 1 of the pair
    v16i magic;
#pragma unroll
    for (int r = 0; r < 16; ++r) magic[r] = kMagic;
    // acc += (I d_w rounded once) d_x for the 16 results of one MFMA (the products first, then
    // the accumulations: no VALU instruction waits on the one before it)
    auto consume = [&](v16f & acc, const v16i & e, float dw, float nm, const uint8_t * D) {
        float dx[16];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            // (output order: register r of half h is column 8 (r / 4) + 4 h + r % 4)
            const float4 v = *reinterpret_cast<const float4 *>(D + h * 64 + 16 * q4);
            dx[4 * q4] = v.x;
            dx[4 * q4 + 1] = v.y;
            dx[4 * q4 + 2] = v.z;
            dx[4 * q4 + 3] = v.w;
        }
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
    const uint32_t nshift = (uint32_t)(4 - 4 * h);            // Q4_0: the lane half's nibble to the high nibble
    const Iq4Regs kr = iq4_regs();                             // IQ4_NL: the codebook in VGPRs
    auto compute = [&](int b, int s) {
        const uint8_t * S = lds + (ks * 2 + b) * kKQStage;
        const uint4 dd = wd;
        const uint32_t sn = (uint32_t)std::min(s + 1, s1 - 1) * tgs;   // the next group (clamped)
        wd = bld16(wbuf, row16, sn + kDch * kChunk);
#pragma unroll
        for (int jb = 0; jb < 8; ++jb) {
            const uint4 x = wq[jb];
            v4i bop;
            if constexpr (Q8) {
                bop = v4i{ (int)x.x, (int)x.y, (int)x.z, (int)x.w };
            } else if constexpr (NLQ) {
                const uint32_t sh = 4u * (uint32_t)h;
                bop = v4i{ (int)iq4_lookup_r(x.x >> sh, kr), (int)iq4_lookup_r(x.y >> sh, kr),
                           (int)iq4_lookup_r(x.z >> sh, kr), (int)iq4_lookup_r(x.w >> sh, kr) };
            } else {
                // (q ^ 8) in the high nibble: the int8 byte is 16 (q - 8)
                bop = v4i{ (int)(((x.x << nshift) & 0xF0F0F0F0u) ^ 0x80808080u),
                           (int)(((x.y << nshift) & 0xF0F0F0F0u) ^ 0x80808080u),
                           (int)(((x.z << nshift) & 0xF0F0F0F0u) ^ 0x80808080u),
                           (int)(((x.w << nshift) & 0xF0F0F0F0u) ^ 0x80808080u) };
            }
            const uint32_t dword = jb < 2 ? dd.x : jb < 4 ? dd.y : jb < 6 ? dd.z : dd.w;
            float dw = h2f((dword >> (16 * (jb & 1))) & 0xffffu);
            asm volatile("" : "+v"(dw));                      // f32 operands (no fp16 source folding)
            const float nm = -12582912.0f * dw;
            const v4i a0 = *reinterpret_cast<const v4i *>(S + jb * 1024 + lane16);
            const v4i a1 = *reinterpret_cast<const v4i *>(S + 8192 + jb * 1024 + lane16);
            const v16i e0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bop, magic, 0, 0, 0);
            const v16i e1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bop, magic, 0, 0, 0);
            wq[jb] = bld16(wbuf, row16, sn + wplane(jb));     // the slot's next group (its registers free)
            consume(out0, e0, dw, nm, S + 16384 + jb * 128);
            consume(out1, e1, dw, nm, S + 17408 + jb * 128);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // ---- K loop: group s + 1 goes into LDS while s is computed (its buffer was last read before
    // the previous barrier); the barrier's wait covers only these LDS loads, which are issued
    // before the iteration's weight loads (9 per lane)
    stage(s0, 0);
#pragma unroll
    for (int jb = 0; jb < 8; ++jb) wq[jb] = bld16(wbuf, row16, (uint32_t)s0 * tgs + wplane(jb));
    wd = bld16(wbuf, row16, (uint32_t)s0 * tgs + kDch * kChunk);
    __syncthreads();
    for (int it = 0; it < sps; ++it) {                        // uniform over the work-group
        const int s = s0 + it;
        stage(std::min(s + 1, s1 - 1), (it + 1) & 1);         // (past the slice: a copy nobody reads)
        __builtin_amdgcn_sched_barrier(0);                    // the LDS loads go out before the weight loads
        if (s < s1) {
            compute(it & 1, s);
        } else {                                              // a slice shorter than sps: the same loads as
#pragma unroll                                                // compute's (unused), so that every path
            for (int jb = 0; jb < 8; ++jb)                    // leaves them outstanding at the barrier
                wq[jb] = bld16(wbuf, row16, (uint32_t)(s1 - 1) * tgs + wplane(jb));
            wd = bld16(wbuf, row16, (uint32_t)(s1 - 1) * tgs + kDch * kChunk);
        }
        // this wave's LDS loads are complete once at most the 9 weight loads issued after them
        // are outstanding (vmcnt(9)); the barrier then publishes them to the other waves
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(kVmcnt9);
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
    const float scale = (TYPE == QMM_TYPE_Q4_0) ? 0.0625f : 1.0f;   // Q4_0 codes carried 16 (q - 8)
    // a tail piece: the block's pieces meet first, the holder of a sum stores it
    const uint32_t live = piece >= 0 ? kq_meet(p.tree + ((size_t)(L - p.full) * U + u) * (size_t)p.tslots * 2048, piece,
                                               p.ts, out0, out1, lane)
                                     : 0xffffffffu;
    float * dst = p.dst + (int64_t)i2 * p.bt.d_nb2 + (int64_t)i3 * p.bt.d_nb3 + m;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int64_t n0 = (2 * (int64_t)nb + c) * 32;
        const v16f & v = c ? out1 : out0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t n = n0 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (n < p.N && ((live >> (16 * c + r)) & 1u)) __builtin_nontemporal_store(v[r] * scale, dst + n * p.bt.d_nb1);
        }
    }
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

template <int U, bool GATHER>
hipError_t launch_q6k(const KQParams & q, const G3Shape & sh, const dim3 & g, const dim3 & b, hipStream_t s,
                      const KTime * kt) {
    static const hipError_t attr = hipFuncSetAttribute((const void *)k_gemm3_q6k<U, GATHER>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    if (kt) hipExtLaunchKernelGGL(k_gemm3_q6k<U, GATHER>, g, b, (uint32_t)sh.lds, s, kt->start, kt->stop, 0, q);
    else k_gemm3_q6k<U, GATHER><<<g, b, sh.lds, s>>>(q);
    return hipGetLastError();
}

template <int TYPE, int U, bool GATHER>
hipError_t launch_sbs(const KQParams & q, const G3Shape & sh, const dim3 & g, const dim3 & b, hipStream_t s,
                      const KTime * kt) {
    static const hipError_t attr = hipFuncSetAttribute((const void *)k_gemm3_sbs<TYPE, U, GATHER>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    if (kt) hipExtLaunchKernelGGL(k_gemm3_sbs<TYPE, U, GATHER>, g, b, (uint32_t)sh.lds, s, kt->start, kt->stop, 0, q);
    else k_gemm3_sbs<TYPE, U, GATHER><<<g, b, sh.lds, s>>>(q);
    return hipGetLastError();
}

template <int TYPE, bool GATHER>
hipError_t launch_sbs_u(const KQParams & q, const G3Shape & sh, const dim3 & g, const dim3 & b, hipStream_t s,
                        const KTime * kt) {
    switch (sh.U) {
        case 12: return launch_sbs<TYPE, 12, GATHER>(q, sh, g, b, s, kt);
        case 6: return launch_sbs<TYPE, 6, GATHER>(q, sh, g, b, s, kt);
        case 4: return launch_sbs<TYPE, 4, GATHER>(q, sh, g, b, s, kt);
        case 3: return launch_sbs<TYPE, 3, GATHER>(q, sh, g, b, s, kt);
        case 2: return launch_sbs<TYPE, 2, GATHER>(q, sh, g, b, s, kt);
        default: return hipErrorInvalidValue;
    }
}

template <bool GATHER>
hipError_t launch_q6k_u(const KQParams & q, const G3Shape & sh, const dim3 & g, const dim3 & b, hipStream_t s,
                        const KTime * kt) {
    switch (sh.U) {
        case 12: return launch_q6k<12, GATHER>(q, sh, g, b, s, kt);
        case 6: return launch_q6k<6, GATHER>(q, sh, g, b, s, kt);
        case 4: return launch_q6k<4, GATHER>(q, sh, g, b, s, kt);
        case 3: return launch_q6k<3, GATHER>(q, sh, g, b, s, kt);
        case 2: return launch_q6k<2, GATHER>(q, sh, g, b, s, kt);
        default: return hipErrorInvalidValue;
    }
}

template <int TYPE, int U>
hipError_t launch_blk(const KQParams & q, const G3Shape & sh, const dim3 & g, const dim3 & b, hipStream_t s,
                      const KTime * kt) {
    static const hipError_t attr = hipFuncSetAttribute((const void *)k_gemm3_blk<TYPE, U>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    if (kt) hipExtLaunchKernelGGL(k_gemm3_blk<TYPE, U>, g, b, (uint32_t)sh.lds, s, kt->start, kt->stop, 0, q);
    else k_gemm3_blk<TYPE, U><<<g, b, sh.lds, s>>>(q);
    return hipGetLastError();
}

template <int TYPE>
hipError_t launch_blk_u(const KQParams & q, const G3Shape & sh, const dim3 & g, const dim3 & b, hipStream_t s,
                        const KTime * kt) {
    switch (sh.U) {
        case 12: return launch_blk<TYPE, 12>(q, sh, g, b, s, kt);
        case 6: return launch_blk<TYPE, 6>(q, sh, g, b, s, kt);
        case 4: return launch_blk<TYPE, 4>(q, sh, g, b, s, kt);
        case 3: return launch_blk<TYPE, 3>(q, sh, g, b, s, kt);
        case 2: return launch_blk<TYPE, 2>(q, sh, g, b, s, kt);
        default: return hipErrorInvalidValue;
    }
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
           (type == QMM_TYPE_Q4_K && env_int3("QMM_GEMM3_Q4K", 1) != 0) ||
           (type == QMM_TYPE_Q6_K && env_int3("QMM_GEMM3_Q6K", 1) != 0) ||
           ((type == QMM_TYPE_Q5_K || type == QMM_TYPE_IQ4_XS) && env_int3("QMM_GEMM3_SBS", 1) != 0);
}

namespace {
// Q4_K launch shape: U row-half waves per K slice x KS slices, chosen by rounds of work-groups
// on the chip x super-blocks per slice: 12-wave work-groups fill a CU alone (3 waves per SIMD),
// whole rounds; 4-wave ones go three to a CU and a partial last round costs its fraction (the
// CUs take the next small group as one finishes; measured on 17408 x 5120 x 512: 4-wave groups
// 141 us, (6, 2) 145 us, (12, 1) 155 us).  Ties go to the earlier (larger U) candidate.
// ncp = column pairs (grouped mode: route units) per batch; tail: a dense launch (its U = 2
// charge and the tail pieces); only >= 0: that candidate alone (the grouped mode's one-slice
// form, kKQOneSlice); only = -2: every candidate but that one (the grouped mode's split form:
// there it tied with (2, 2, 3) on 128 experts x 32 pairs and measured 54.8 against 46.8 us)
constexpr int kKQOneSlice = 4;                                // (4, 1, 3) in the candidates below
bool kq_shape_ncp(const WView & w, int64_t ncp, int64_t nbatch, G3Shape * sh, bool blk, bool tail, int only) {
    struct Cand { int U, KS, per_cu; };
    static const Cand cands[] = { { 12, 1, 1 }, { 6, 2, 1 }, { 4, 3, 1 }, { 3, 4, 1 }, { 4, 1, 3 }, { 2, 2, 3 } };
    const int64_t nrh = 2 * w.ntiles, G = w.G;
    const int cus = 256;
    int64_t best = -1;
    const int forced = env_int3("QMM_GEMM3_KQ", -1);           // index into cands (tuning)
    for (int i = 0; i < (int)(sizeof(cands) / sizeof(cands[0])); ++i) {
        if (forced >= 0 && i != forced) continue;
        if (forced < 0 && only >= 0 && i != only) continue;
        if (forced < 0 && only == -2 && i == kKQOneSlice) continue;
        const Cand & c = cands[i];
        // (the block types: two waves per stage share too little of their 2 KB of activations per
        // block; 11008 x 4096 x 512 measured 97 us at (2, 2) against 76 at (12, 1) and (4, 1, 3))
        if (blk && c.U == 2 && forced < 0) continue;
        const int64_t sps = (G + c.KS - 1) / c.KS, KS = (G + sps - 1) / sps;
        const int64_t mbn = (nrh + c.U - 1) / c.U, nwg = mbn * ncp * nbatch;
        const int64_t slots = (int64_t)cus * c.per_cu;
        // (in 1/64 rounds)
        const int64_t rounds = c.per_cu > 1 ? std::max<int64_t>(64, (nwg * 64 + slots - 1) / slots)
                                            : 64 * ((nwg + slots - 1) / slots);
        // (dense launches: two row-half waves share a stage of activations, half the sharing of
        // four, a cost the rounds do not count: U = 2 pays 1/16 more.  Q6_K 151936 x 5120 x 512 tied
        // (2, 2, 3) with (4, 1, 3) to rounding and measured 1.50 against 1.33 ms)
        const int64_t cost = tail && c.U == 2 ? rounds * sps * 17 / 16 : rounds * sps;
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
    // The blocks past a whole number per CU (one K slice, one batch) run as ts pieces along K.
    // The hardware puts a block where one finishes, so each CU runs nwg / CUs whole blocks and
    // the remainder would keep nwg % CUs CUs a whole block longer than the rest.  ts minimizes
    // the pieces' load per CU, ceil(tail ts / CUs) / ts blocks, below the one block; at least two
    // stages a piece, ties to fewer pieces.  (Measured at N = 512: IQ4_NL 14336 x 4096, 896
    // blocks of 4 waves = 3 x 256 + 128, 124 -> 108 us in halves.  Q4_K 17408 x 5120, 1088
    // blocks = 4 x 256 + 64: a per-block timeline showed each CU's three resident blocks served
    // oldest first at a steady ~24 us of CU time per block, 192 CUs done at ~100 us and the 64
    // with a fifth block at ~120.)
    const int64_t nwg = sh->mbn * ncp;
    sh->full = nwg;
    sh->ts = 1;
    sh->pk = (int)G;
    sh->tslots = 0;
    const int tail_env = env_int3("QMM_GEMM3_TAIL", 1);       // 0: whole blocks, 2..4: that many pieces (tuning)
    if (tail && nbatch == 1 && sh->KS == 1 && tail_env != 0) {
        const int64_t full = nwg / cus * cus, rest = nwg - full;
        int64_t bn = 1, bd = 1;                                 // best load bn / bd (1: whole blocks)
        for (int ts = 2; ts <= 4 && rest > 0 && (rest <= cus || tail_env > 1); ++ts) {
            const int64_t pk = (G + ts - 1) / ts;
            if (pk < 2 || (ts - 1) * pk >= G || (tail_env > 1 && ts != tail_env)) continue;
            const int64_t r = (rest * ts + cus - 1) / cus;
            if (r * bd < bn * ts || tail_env > 1) {
                bn = r;
                bd = ts;
            }
        }
        if (bd > 1) {
            sh->full = full;
            sh->ts = (int)bd;
            sh->pk = (int)((G + bd - 1) / bd);
            sh->tslots = bd == 2 ? 1 : 3;                       // (pairs, then the pair of pairs)
        }
    }
    sh->fchunk = (sh->full + 7) / 8;
    sh->tchunk = ((nwg - sh->full) * sh->ts + 7) / 8;
    sh->workgroups = 8 * (sh->fchunk + sh->tchunk) * nbatch;
    return sh->mbn * ncp < 0x7fffffff && sh->lds <= 160 * 1024 && sh->threads <= 64 * kKQMaxWaves;
}
bool kq_shape(const WView & w, int64_t N, int64_t nbatch, G3Shape * sh, bool blk) {
    return kq_shape_ncp(w, ((N + 31) / 32 + 1) / 2, nbatch, sh, blk, true, -1);
}
}  // namespace

bool gemm3_id_supported(int type) {
    return (type == QMM_TYPE_Q4_K || type == QMM_TYPE_Q6_K || type == QMM_TYPE_Q5_K || type == QMM_TYPE_IQ4_XS) &&
           gemm3_supported(type);
}

bool gemm3_id_shape(const WView & w, int64_t max_units, bool one_slice, G3Shape * sh) {
    return max_units > 0 && w.G > 0 && w.ntiles > 0 &&
           kq_shape_ncp(w, max_units, 1, sh, false, false, one_slice ? kKQOneSlice : -2);
}

hipError_t launch_gemm3_id(int type, const WView & w, const ActBuf & a, const GemmUnit * units, const int32_t * nunits,
                           int64_t max_units, bool one_slice, float * dst, int64_t dst_span, hipStream_t s,
                           const KTime * kt, const float * gsrc, int glu) {
    G3Shape sh;
    if (!gemm3_id_supported(type) || a.vdt != QMM_TYPE_Q8_K || !a.bsp || !units || !nunits || a.ldk != w.G * 256 ||
        dst_span <= 0 || dst_span >= ((int64_t)1 << 30) ||
        (glu >= 0) != (gsrc != nullptr) ||
        (glu != -1 && glu != QMM_GLU_REGLU && glu != QMM_GLU_GEGLU && glu != QMM_GLU_SWIGLU &&
         glu != QMM_GLU_GEGLU_ERF && glu != QMM_GLU_GEGLU_QUICK) ||
        !gemm3_id_shape(w, max_units, one_slice, &sh) || a.ncols * a.ldk >= ((int64_t)1 << 31) ||
        w.G * a.ldT * 16 >= ((int64_t)1 << 31) || a.ldT < a.ncols)
        return hipErrorInvalidValue;
    KQParams q{};
    q.w = w;
    q.nsb = w.G;
    q.mbn = sh.mbn;
    q.nbn = max_units;
    q.total = sh.mbn * max_units;
    q.full = q.total;
    q.fchunk = (q.total + 7) / 8;
    q.ts = 1;
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
    q.gsrc = gsrc;
    q.glu = glu;
    q.dspan = dst_span;
    const dim3 g((unsigned)(8 * q.fchunk), 1u), b(sh.threads);
    switch (type) {
        case QMM_TYPE_Q4_K: return launch_kq_u<true>(q, sh, g, b, s, kt);
        case QMM_TYPE_Q6_K: return launch_q6k_u<true>(q, sh, g, b, s, kt);
        case QMM_TYPE_Q5_K: return launch_sbs_u<QMM_TYPE_Q5_K, true>(q, sh, g, b, s, kt);
        case QMM_TYPE_IQ4_XS: return launch_sbs_u<QMM_TYPE_IQ4_XS, true>(q, sh, g, b, s, kt);
        default: return hipErrorInvalidValue;
    }
}

// Launch shape of both kernels (kq_shape): U row-half waves per K slice x KS slices.
bool gemm3_shape(int type, const WView & w, int64_t N, int64_t nbatch, G3Shape * sh) {
    if (!gemm3_supported(type) || N <= 0 || nbatch <= 0 || nbatch > 65535 || w.G <= 0 || w.ntiles <= 0) return false;
    // (the K-quant frame's launch rule for the super-block types; the block types' for the rest)
    const bool kframe = type == QMM_TYPE_Q4_K || type == QMM_TYPE_Q6_K || type == QMM_TYPE_Q5_K || type == QMM_TYPE_IQ4_XS;
    return kq_shape(w, N, nbatch, sh, !kframe);
}

size_t gemm3_tree_words(const G3Shape & sh) {
    return sh.ts > 1 ? (size_t)(sh.mbn * sh.nbn - sh.full) * (size_t)sh.U * (size_t)sh.tslots * 2048 : 0;
}

hipError_t launch_gemm3(int type, const WView & w, const TiledAct & a, int64_t nbatch, const GemmBatch & bt,
                        float * dst, hipStream_t s, const KTime * kt, uint32_t * tree) {
    G3Shape sh;
    if (!gemm3_shape(type, w, a.N, nbatch, &sh) || !a.A || !a.D || a.nblk != w.G * 8 || a.ntb != (a.N + 31) / 32 ||
        a.ntiles != a.ntb * nbatch || a.vdt != vec_dot_type(type))
        return hipErrorInvalidValue;
    if ((type == QMM_TYPE_Q4_K || type == QMM_TYPE_Q5_K) && !a.S) return hipErrorInvalidValue;
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
    q.U = sh.U;
    q.KS = sh.KS;
    q.sps = sh.sps;
    q.bt = bt;
    q.dst = dst;
    if (sh.ts > 1 && tree) {                                  // the tail in pieces
        q.full = sh.full;
        q.fchunk = sh.fchunk;
        q.tchunk = sh.tchunk;
        q.ts = sh.ts;
        q.pk = sh.pk;
        q.tslots = sh.tslots;
        q.tree = tree;
    } else {
        q.full = q.total;
        q.fchunk = (q.total + 7) / 8;
        q.ts = 1;
    }
    const dim3 g((unsigned)(8 * (q.fchunk + q.tchunk)), (unsigned)nbatch), b(sh.threads);
    switch (type) {
        case QMM_TYPE_Q4_K: return launch_kq_u<false>(q, sh, g, b, s, kt);
        case QMM_TYPE_Q6_K: return launch_q6k_u<false>(q, sh, g, b, s, kt);
        case QMM_TYPE_Q5_K: return launch_sbs_u<QMM_TYPE_Q5_K, false>(q, sh, g, b, s, kt);
        case QMM_TYPE_IQ4_XS: return launch_sbs_u<QMM_TYPE_IQ4_XS, false>(q, sh, g, b, s, kt);
        case QMM_TYPE_Q4_0: return launch_blk_u<QMM_TYPE_Q4_0>(q, sh, g, b, s, kt);
        case QMM_TYPE_Q8_0: return launch_blk_u<QMM_TYPE_Q8_0>(q, sh, g, b, s, kt);
        case QMM_TYPE_IQ4_NL: return launch_blk_u<QMM_TYPE_IQ4_NL>(q, sh, g, b, s, kt);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
