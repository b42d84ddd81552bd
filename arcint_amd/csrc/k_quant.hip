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

// q8_0 into the streaming GEMM's tiled layout: 8 lanes per 32-weight block, 4 weights per
// lane, over every column of every tile (columns past N of a batch quantize zeros, which gives
// zero codes and a zero scale)
__global__ void k_quant_tiled_q8_0(F32Cols src, int64_t K, TiledAct ta, int64_t nthreads) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = t < nthreads;                // whole waves are live or dead
    const int64_t kq = ta.nblk * 8;                // threads per column
    const int64_t cp = live ? t / kq : 0, k = live ? (t - cp * kq) * 4 : 0;
    const int64_t tile = cp >> 5, b = tile / ta.ntb;
    const int i = (int)(cp & 31);
    const int64_t n = (tile - b * ta.ntb) * 32 + i;
    float v[4] = { 0.f, 0.f, 0.f, 0.f };
    if (live && n < ta.N && k < K) {
        const float * x = f32_col(src, b * ta.N + n) + k;
        for (int j = 0; j < 4; ++j) v[j] = x[j];
    }
    float d;
    int s;
    const uint32_t packed = quant_q8_0_lane(v, &d, &s);
    if (!live) return;
    const int64_t blk = tile * ta.nblk + (k >> 5);
    const int o = (int)(k & 31);
    *reinterpret_cast<uint32_t *>(ta.A + ((blk * 64 + (o >> 4) * 32 + i) << 4) + (o & 15)) = packed;
    if ((t & 7) == 0) ta.D[blk * 32 + tiled_pos(i)] = d;
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
        t.N > 32 * t.ntb)
        return hipErrorInvalidValue;
    const int64_t n = t.ntiles * 32 * t.nblk * 8;    // a multiple of 64: whole waves
    const int64_t grid = (n + kTpb - 1) / kTpb;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    k_quant_tiled_q8_0<<<dim3((unsigned)grid), kTpb, 0, s>>>(src, K, t, n);
    return hipGetLastError();
}

hipError_t launch_act_to_blocks(const ActBuf & a, void * out, hipStream_t s) {
    const int64_t nb = a.ncols * (a.K / act_block(a.vdt));
    if (nb <= 0) return hipSuccess;
    k_act_blocks<<<dim3((unsigned)((nb + 255) / 256)), 256, 0, s>>>(a, (uint8_t *)out);
    return hipGetLastError();
}

}  // namespace qmm
