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
    int64_t mr, i1, i2;
    const int64_t c = qdiv(t, rows, mr), m = z.m0 + mr;
    const int64_t r = qdiv(c, z.ne1, i1), i3 = qdiv(r, z.ne2, i2);
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
    int64_t blk, tt;
    const int64_t tile = qdiv(w, ta.nblk, blk), b = qdiv(tile, ta.ntb, tt);
    const int64_t n = tt * 32 + i, k0 = blk * 32 + 16 * h;
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

// q8_K into the tiled layout: one work-group of 8 waves per (tile, 256-weight super-block),
// wave w the super-block's sub-block w; lane (i, h) holds k 16 h .. 16 h + 15 of it in column
// i of the tile (columns past N of a batch quantize zeros).  quantize_row_q8_K_ref's scale
// source is the first element of the largest |x| (a strictly larger |x| replaces it, scanning
// k upwards): each lane finds its own first maximum, the two lane halves of a wave (k ranges
// 16 h + [0, 16) of the same sub-block) and then the 8 waves (sub-blocks in k order, through
// LDS) keep the earlier one on ties.  iscale, the codes and d follow quant_q8_K_wave's
// arithmetic step for step.  Writes: the codes as the 1 KB A operand of block sb * 8 + w, the
// super-block's d into D in output order, and each sub-block's code sum split as 64 bh + bl
// into S (column i: bh[8], then bl[8]).
__global__ __launch_bounds__(512) void k_quant_tiled_q8_K(F32Cols src, int64_t K, TiledAct ta, int64_t nsb) {
    __shared__ float s_amax[8][32], s_mx[8][32];
    __shared__ int8_t s_split[32][16];
    const int64_t job = blockIdx.x;                  // (tile, super-block)
    int64_t sb, tt;
    const int64_t tile = qdiv(job, nsb, sb), b = qdiv(tile, ta.ntb, tt);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
    const int64_t n = tt * 32 + i, k0 = sb * 256 + 32 * w + 16 * h;
    float v[16];
    if (n < ta.N && k0 < K) {
        const float * x = f32_col(src, b * ta.N + n) + k0;   // (column strides are only 4-byte aligned)
#pragma unroll
        for (int q = 0; q < 16; ++q) v[q] = x[q];
    } else {
#pragma unroll
        for (int q = 0; q < 16; ++q) v[q] = 0.0f;
    }
    float am = 0.0f, mx = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const float a = fabsf(v[q]);
        if (a > am) {
            am = a;
            mx = v[q];
        }
    }
    // the other lane half of the same column (h = 0 holds the lower k)
    const auto sa = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, am), __builtin_bit_cast(uint32_t, am),
                                                     false, false);
    const auto sm = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, mx), __builtin_bit_cast(uint32_t, mx),
                                                     false, false);
    const float oam = __builtin_bit_cast(float, h ? sa[0] : sa[1]), omx = __builtin_bit_cast(float, h ? sm[0] : sm[1]);
    float wam, wmx;                                  // the sub-block's first maximum
    if (h == 0) {
        wam = oam > am ? oam : am;
        wmx = oam > am ? omx : mx;
    } else {
        wam = am > oam ? am : oam;
        wmx = am > oam ? mx : omx;
    }
    if (h == 0) {
        s_amax[w][i] = wam;
        s_mx[w][i] = wmx;
    }
    __syncthreads();
    float amax = s_amax[0][i], m = s_mx[0][i];
#pragma unroll
    for (int u = 1; u < 8; ++u) {
        const float a = s_amax[u][i];
        if (a > amax) {
            amax = a;
            m = s_mx[u][i];
        }
    }
    int c[16];
    float dv = 0.0f;
    if (amax != 0.0f) {
        const float iscale = -127.f / m;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int r = (int)__builtin_rintf(iscale * v[q]);
            c[q] = r > 127 ? 127 : r;
        }
        dv = 1.0f / iscale;
    } else {
#pragma unroll
        for (int q = 0; q < 16; ++q) c[q] = 0;
    }
    uint32_t word[4];
    int s16 = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        word[q] = (uint32_t)(c[4 * q] & 0xff) | ((uint32_t)(c[4 * q + 1] & 0xff) << 8) |
                  ((uint32_t)(c[4 * q + 2] & 0xff) << 16) | ((uint32_t)(c[4 * q + 3] & 0xff) << 24);
        s16 += c[4 * q] + c[4 * q + 1] + c[4 * q + 2] + c[4 * q + 3];
    }
    const int64_t blk = tile * ta.nblk + sb * 8 + w;
    *reinterpret_cast<uint4 *>(ta.A + (blk * 64 + lane) * 16) = make_uint4(word[0], word[1], word[2], word[3]);
    const auto ss = __builtin_amdgcn_permlane32_swap((uint32_t)s16, (uint32_t)s16, false, false);
    const int s32 = s16 + (int)(h ? ss[0] : ss[1]);
    if (h == 0) {
        s_split[i][w] = (int8_t)(s32 >> 6);
        s_split[i][8 + w] = (int8_t)(s32 & 63);
    }
    __syncthreads();
    if (w == 0 && h == 0) {
        const int64_t t = tile * (ta.nblk / 8) + sb;
        *reinterpret_cast<uint4 *>(ta.S + (t * 32 + i) * 16) = *reinterpret_cast<const uint4 *>(&s_split[i][0]);
        ta.D[t * 32 + tiled_pos(i)] = dv;
    }
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
    if (t.vdt == QMM_TYPE_Q8_K) {
        if (K % 256 || !t.S) return hipErrorInvalidValue;
        const int64_t nsb = t.nblk / 8, grid = t.ntiles * nsb;
        if (grid > 0x7fffffff) return hipErrorInvalidValue;
        k_quant_tiled_q8_K<<<dim3((unsigned)grid), 512, 0, s>>>(src, K, t, nsb);
        return hipGetLastError();
    }
    if (t.vdt != QMM_TYPE_Q8_0) return hipErrorInvalidValue;
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
