// k_quant.hip - activation quantization on gfx950, bit-exact with ggml-cpu's
// from_float for the vec_dot type:
//   q8_0  x86 quantize_row_q8_0 (restated at 0000-03-...patch:646-669):
//         d = fp16(amax / 127), codes = round-half-even(x * (127 / amax))
//   q8_K  quantize_row_q8_K_ref (restated at 0000-03-...patch:673-683):
//         mx = first element of largest |x|, iscale = -127 / mx,
//         codes = min(127, round-half-even(iscale * x)), d = 1 / iscale,
//         bsums = sums of 16 codes; an all-zero block stays zero.
// Divisions are IEEE (hipcc's default correctly-rounded f32 divide) and no
// multiply is contracted, so every code and scale equals the CPU's.
// Columns are written with a stride of ldk (K rounded up to 256); the padding
// past K quantizes zeros.  For a GEMM consumer the scales are written again
// block-major (dT); for q8_K the sub-block sums are also written split into
// int8 halves (bsp), the int8 MFMA operand of the Q4_K min term in the GEMM
// and the few-column GEMV.  The same launch can zero dst columns for a GEMV
// that adds its K slices with atomics (work-groups past the quantization
// ones do that).
#include "qmm_device.h"

namespace qmm {
namespace {

#pragma clang fp contract(off)

constexpr int kTpb = 256;

__device__ void zero_cols(const ZeroJob & z, int64_t t) {
    const int64_t rows = z.M - z.m0, n = rows * z.ncols;
    if (t >= n) return;
    const int64_t c = t / rows, m = z.m0 + (t - c * rows);
    const int64_t r = c / z.ne1, i1 = c - r * z.ne1, i3 = r / z.ne2, i2 = r - i3 * z.ne2;
    z.dst[i1 * z.nb1 + i2 * z.nb2 + i3 * z.nb3 + m] = 0.0f;
}

// 8 lanes per 32-weight block, 4 weights per lane
__global__ void k_quant_q8_0(F32Cols src, int64_t K, int64_t ncols, ActBuf a, ZeroJob z, int64_t nqblk) {
    if ((int64_t)blockIdx.x >= nqblk) {
        zero_cols(z, ((int64_t)blockIdx.x - nqblk) * kTpb + threadIdx.x);
        return;
    }
    quant_q8_0_at(src, K, ncols, a, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

// one wave per 256-weight super-block, 4 weights per lane
__global__ void k_quant_q8_K(F32Cols src, int64_t K, int64_t ncols, ActBuf a, ZeroJob z, int64_t nqblk) {
    if ((int64_t)blockIdx.x >= nqblk) {
        zero_cols(z, ((int64_t)blockIdx.x - nqblk) * kTpb + threadIdx.x);
        return;
    }
    quant_q8_K_at(src, K, ncols, a, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

// q8_0 into the streaming GEMM's tiled layout: one wave per (tile, 32-weight block), lane
// (i, h) quantizes k 16 h .. 16 h + 15 of the block in column i of the tile (columns past N
// of a batch quantize zeros: zero codes and a zero scale).  The block's |x| maximum meets the
// other half's through v_permlane32_swap; the scale and the codes follow quant_q8_0_lane's
// arithmetic step for step (the same bits).  Each lane writes its 16 codes as one chunk, so a
// wave writes the block's 1 KB A operand in one piece.
__global__ __launch_bounds__(256) void k_quant_tiled_q8_0(F32Cols src, int64_t K, TiledAct ta, int64_t nwaves) {
    const int64_t w = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    if (w >= nwaves) return;                       // whole waves
    const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
    const int64_t tile = w / ta.nblk, blk = w - tile * ta.nblk, b = tile / ta.ntb;
    const int64_t n = (tile - b * ta.ntb) * 32 + i, k0 = blk * 32 + 16 * h;
    float v[16];
    if (n < ta.N && k0 < K) {
        const float * x = f32_col(src, b * ta.N + n) + k0;   // (column strides are only 4-byte aligned)
#pragma unroll
        for (int q = 0; q < 16; ++q) v[q] = x[q];
    } else {
#pragma unroll
        for (int q = 0; q < 16; ++q) v[q] = 0.0f;
    }
    float m = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) m = fmaxf(m, fabsf(v[q]));
    const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, m), __builtin_bit_cast(uint32_t, m),
                                                     false, false);
    const float amax = fmaxf(m, __builtin_bit_cast(float, h ? sw[0] : sw[1]));
    const _Float16 dh = (_Float16)(amax / 127.f);
    const float mul = amax != 0.0f ? 127.f / amax : 0.0f;
    uint32_t c[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float r = __builtin_rintf(v[4 * q + e] * mul);
            r = fminf(fmaxf(r, -128.f), 127.f);
            word |= ((uint32_t)(int)r & 0xffu) << (8 * e);
        }
        c[q] = word;
    }
    const int64_t t = tile * ta.nblk + blk;
    *reinterpret_cast<uint4 *>(ta.A + (t * 64 + lane) * 16) = make_uint4(c[0], c[1], c[2], c[3]);
    if (h == 0) ta.D[t * 32 + tiled_pos(i)] = (float)dh;
}

// ActBuf -> ggml block bytes, one thread per block
__global__ void k_act_blocks(ActBuf a, uint8_t * __restrict__ out) {
    const int bs = act_block(a.vdt);
    const int64_t nbc = a.K / bs, nb = a.ncols * nbc;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nb) return;
    const int64_t c = i / nbc, b = i - c * nbc;
    const int8_t * codes = a.codes + c * a.ldk + b * bs;
    const float d = a.d[c * (a.ldk / bs) + b];
    if (a.vdt == QMM_TYPE_Q8_0) {
        uint8_t * o = out + i * 34;
        const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)d);
        o[0] = (uint8_t)(h & 0xff);
        o[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; ++j) o[2 + j] = (uint8_t)codes[j];
    } else {
        uint8_t * o = out + i * 292;
        const uint32_t db = __builtin_bit_cast(uint32_t, d);
        for (int j = 0; j < 4; ++j) o[j] = (uint8_t)(db >> (8 * j));
        for (int j = 0; j < 256; ++j) o[4 + j] = (uint8_t)codes[j];
        const int16_t * sums = a.sums + c * (a.ldk / 16) + b * 16;
        for (int j = 0; j < 16; ++j) {
            const uint16_t v = (uint16_t)sums[j];
            o[260 + 2 * j] = (uint8_t)(v & 0xff);
            o[261 + 2 * j] = (uint8_t)(v >> 8);
        }
    }
}

}  // namespace

hipError_t launch_quantize(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, const ZeroJob * z,
                           hipStream_t s) {
    if (K <= 0 || a.ldk % 256 || a.ldk < K) return hipErrorInvalidValue;
    const ZeroJob zj = z ? *z : ZeroJob{};
    const int64_t nzblk = z ? ((zj.M - zj.m0) * zj.ncols + kTpb - 1) / kTpb : 0;
    int64_t nq = a.vdt == QMM_TYPE_Q8_0 ? ncols * (a.ldk / 4) : ncols * (a.ldk / 256) * 64;
    const int64_t nqblk = ncols > 0 ? (nq + kTpb - 1) / kTpb : 0;
    const int64_t grid = nqblk + nzblk;
    if (grid <= 0) return hipSuccess;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    if (a.vdt == QMM_TYPE_Q8_0) k_quant_q8_0<<<dim3((unsigned)grid), kTpb, 0, s>>>(src, K, ncols, a, zj, nqblk);
    else k_quant_q8_K<<<dim3((unsigned)grid), kTpb, 0, s>>>(src, K, ncols, a, zj, nqblk);
    return hipGetLastError();
}

hipError_t launch_quantize_tiled(const F32Cols & src, int64_t K, const TiledAct & t, hipStream_t s) {
    if (K <= 0 || t.nblk * 32 < K || t.nblk % 8 || t.ntb <= 0 || t.ntiles <= 0 || t.ntiles % t.ntb || t.N <= 0 ||
        t.N > 32 * t.ntb || K % 32)
        return hipErrorInvalidValue;
    const int64_t nw = t.ntiles * t.nblk, grid = (nw + 3) / 4;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    k_quant_tiled_q8_0<<<dim3((unsigned)grid), 256, 0, s>>>(src, K, t, nw);
    return hipGetLastError();
}

hipError_t launch_act_to_blocks(const ActBuf & a, void * out, hipStream_t s) {
    const int64_t nb = a.ncols * (a.K / act_block(a.vdt));
    if (nb <= 0) return hipSuccess;
    k_act_blocks<<<dim3((unsigned)((nb + 255) / 256)), 256, 0, s>>>(a, (uint8_t *)out);
    return hipGetLastError();
}

}  // namespace qmm
