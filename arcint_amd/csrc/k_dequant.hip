// k_dequant.hip - dequantize_row_* of ggml on gfx950, bit-exact, reading the
// tiled weight image (qmm_internal.h).
//
// Each thread expands one 32-weight group (one 64-weight chunk for Q4_K) of
// one GGUF block in the evaluation order of ggml's dequantize_row_* (restated
// in tools/mtp_fit.py:360-409; kernel forms at P02:2956-2984 (Q4_0),
// P02:4359-4378 (Q8_0), P01:2199-2247 (Q4_K, Q6_K), P01:3390-3398 (IQ4_XS),
// P01:3736-3750 (Q5_K's fifth bits), P01:3414-3455 (IQ4_NL)).
// Every product here is exact in fp32 except the last multiply (Q6_K,
// IQ4_XS) or the last subtract (Q4_K), so contraction is switched off to
// keep that single rounding where ggml has it.
#include "qmm_device.h"

namespace qmm {
namespace {

#pragma clang fp contract(off)

// Where GGUF block b (row-major over all matrices) lives: its tile-group and
// the row r inside the tile; *slot is the block's slot in a 256-weight group.
__device__ __forceinline__ const uint8_t * block_tg(const WView & w, int bpg, int64_t b, int * r, int * slot) {
    const int64_t R = b / w.bpr, kb = b - R * w.bpr;
    const int64_t mat = R / w.M, m = R - mat * w.M;
    *r = (int)(m % kTileRows);
    *slot = (int)(kb % bpg);
    return tile_group(w, mat, m / kTileRows, kb / bpg);
}

__global__ void k_deq_q4_0(WView w, int64_t nblk, float * __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    int r, p;
    const uint8_t * tg = block_tg(w, 8, i, &r, &p);
    const uint4 q = ld16(tg + p * kChunk + r * 16);
    const float d = h2f(*reinterpret_cast<const uint16_t *>(tg + 8 * kChunk + r * 16 + 2 * p));
    const uint32_t qs[4] = { q.x, q.y, q.z, q.w };
    float * o = y + i * 32;
    for (int j = 0; j < 16; ++j) {
        const uint32_t b = (qs[j >> 2] >> (8 * (j & 3))) & 0xffu;
        o[j]      = (float)((int)(b & 0xfu) - 8) * d;
        o[j + 16] = (float)((int)(b >> 4) - 8) * d;
    }
}

__global__ void k_deq_q8_0(WView w, int64_t nblk, float * __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    int r, p;
    const uint8_t * tg = block_tg(w, 8, i, &r, &p);
    const int8_t * q0 = reinterpret_cast<const int8_t *>(tg + (2 * p) * kChunk + r * 16);
    const int8_t * q1 = reinterpret_cast<const int8_t *>(tg + (2 * p + 1) * kChunk + r * 16);
    const float d = h2f(*reinterpret_cast<const uint16_t *>(tg + 16 * kChunk + r * 16 + 2 * p));
    float * o = y + i * 32;
    for (int j = 0; j < 16; ++j) o[j] = (float)q0[j] * d;
    for (int j = 0; j < 16; ++j) o[16 + j] = (float)q1[j] * d;
}

// thread = (block, chunk c of 64 weights)
__global__ void k_deq_q4_K(WView w, int64_t nblk, float * __restrict__ y) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk * 4) return;
    const int64_t i = t >> 2;
    const int c = (int)(t & 3);
    int r, p;
    const uint8_t * tg = block_tg(w, 1, i, &r, &p);
    const uint8_t * b = tg + 8 * kChunk + r * 16;       // header {d, dmin, scales[12]}
    const float d = h2f(reinterpret_cast<const uint16_t *>(b)[0]);
    const float dmin = h2f(reinterpret_cast<const uint16_t *>(b)[1]);
    const uint8_t * s = b + 4;
    int sc[2], m[2];
    for (int h = 0; h < 2; ++h) {
        const int j = (2 * c + h) ^ (QMM_RED == 1);           // (mutation 1, Q4_K: the neighbouring sub-block's scale)
        if (j < 4) { sc[h] = s[j] & 63; m[h] = s[j + 4] & 63; }
        else { sc[h] = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4); m[h] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4); }
    }
    const float d1 = d * (float)sc[0], m1 = dmin * (float)m[0];
    const float d2 = d * (float)sc[1], m2 = dmin * (float)m[1];
    float * o = y + i * 256 + 64 * c;
    for (int l = 0; l < 32; ++l) {                      // qs[32c + l]: chunk 2c + l / 16
        const uint8_t q = tg[(2 * c + (l >> 4)) * kChunk + r * 16 + (l & 15)];
        o[l] = d1 * (float)(q & 0xF) - m1;
        o[32 + l] = d2 * (float)(q >> 4) - m2;
    }
}

// Q5_K: Q4_K's chunk with the fifth bits of qh[l] (chunk 9 + l / 16): bit 2c for the low
// nibble, 2c + 1 for the high one (ggml's dequantize_row_q5_K; the reference's decode of the
// same fields, P01:3736-3750)
__global__ void k_deq_q5_K(WView w, int64_t nblk, float * __restrict__ y) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk * 4) return;
    const int64_t i = t >> 2;
    const int c = (int)(t & 3);
    int r, p;
    const uint8_t * tg = block_tg(w, 1, i, &r, &p);
    const uint8_t * b = tg + 8 * kChunk + r * 16;       // header {d, dmin, scales[12]}
    const float d = h2f(reinterpret_cast<const uint16_t *>(b)[0]);
    const float dmin = h2f(reinterpret_cast<const uint16_t *>(b)[1]);
    const uint8_t * s = b + 4;
    int sc[2], m[2];
    for (int h = 0; h < 2; ++h) {
        const int j = 2 * c + h;
        if (j < 4) { sc[h] = s[j] & 63; m[h] = s[j + 4] & 63; }
        else { sc[h] = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4); m[h] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4); }
    }
    const float d1 = d * (float)sc[0], m1 = dmin * (float)m[0];
    const float d2 = d * (float)sc[1], m2 = dmin * (float)m[1];
    float * o = y + i * 256 + 64 * c;
    for (int l = 0; l < 32; ++l) {
        const uint8_t q = tg[(2 * c + (l >> 4)) * kChunk + r * 16 + (l & 15)];
        const uint8_t qh = tg[(9 + (l >> 4)) * kChunk + r * 16 + (l & 15)];
        o[l] = d1 * (float)((q & 0xF) | (((qh >> (2 * c)) & 1) << 4)) - m1;
        o[32 + l] = d2 * (float)((q >> 4) | (((qh >> (2 * c + 1)) & 1) << 4)) - m2;
    }
}

// IQ4_NL: Q4_0's placement, the codes through the codebook (ggml's dequantize_row_iq4_nl;
// the reference's mv_iq4_nl, P01:3414-3455)
__global__ void k_deq_iq4_nl(WView w, int64_t nblk, float * __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    int r, p;
    const uint8_t * tg = block_tg(w, 8, i, &r, &p);
    const uint8_t * qs = tg + p * kChunk + r * 16;
    const float d = h2f(*reinterpret_cast<const uint16_t *>(tg + 8 * kChunk + r * 16 + 2 * p));
    float * o = y + i * 32;
    for (int j = 0; j < 16; ++j) {
        o[j]      = d * (float)kKvalues[qs[j] & 0xF];
        o[j + 16] = d * (float)kKvalues[qs[j] >> 4];
    }
}

// thread = (block, 32-weight group 32g + l within half n)
__global__ void k_deq_q6_K(WView w, int64_t nblk, float * __restrict__ y) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk * 8) return;
    const int64_t i = t >> 3;
    const int grp = (int)(t & 7), n = grp >> 2, g = grp & 3;
    int r, p;
    const uint8_t * tg = block_tg(w, 1, i, &r, &p);
    const int8_t * sc = reinterpret_cast<const int8_t *>(tg + 12 * kChunk + r * 16) + 8 * n + 2 * g;
    const float d = h2f(*reinterpret_cast<const uint16_t *>(tg + 13 * kChunk + r * 2));
    float * o = y + i * 256 + 128 * n + 32 * g;
    for (int l = 0; l < 32; ++l) {
        const int qlb = 64 * n + 32 * (g & 1) + l, qhb = 32 * n + l;      // byte indices in ql[128], qh[64]
        const uint8_t ql = tg[(qlb >> 4) * kChunk + r * 16 + (qlb & 15)];
        const uint8_t qh = tg[(8 + (qhb >> 4)) * kChunk + r * 16 + (qhb & 15)];
        const int lo = (g < 2) ? (ql & 0xF) : (ql >> 4);
        const int q = lo | (((qh >> (2 * g)) & 3) << 4);
        o[l] = d * (float)sc[l >> 4] * (float)(q - 32);
    }
}

// thread = (block, 32-weight sub-block ib)
__global__ void k_deq_iq4_xs(WView w, int64_t nblk, float * __restrict__ y) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk * 8) return;
    const int64_t i = t >> 3;
    const int ib = (int)(t & 7);
    int r, p;
    const uint8_t * tg = block_tg(w, 1, i, &r, &p);
    const uint8_t * hdr = tg + 8 * kChunk + r * 8;       // {d, scales_h, scales_l[4]}
    const float d = h2f(reinterpret_cast<const uint16_t *>(hdr)[0]);
    const uint32_t sh = reinterpret_cast<const uint16_t *>(hdr)[1];
    const int ls = ((hdr[4 + ib / 2] >> (4 * (ib & 1))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4);
    const float dl = d * (float)(ls - 32);
    const uint8_t * qs = tg + ib * kChunk + r * 16;
    float * o = y + i * 256 + 32 * ib;
    for (int j = 0; j < 16; ++j) {
        o[j]      = dl * (float)kKvalues[qs[j] & 0xF];
        o[j + 16] = dl * (float)kKvalues[qs[j] >> 4];
    }
}

}  // namespace

hipError_t launch_dequant(int type, const WView & w, int64_t nmat, float * y, hipStream_t s) {
    const int64_t nblk = nmat * w.M * w.bpr;
    if (nblk <= 0) return hipSuccess;
    const int tpb = 256;
    auto grid = [&](int64_t n) { return dim3((unsigned)((n + tpb - 1) / tpb)); };
    switch (type) {
        case QMM_TYPE_Q4_0:   k_deq_q4_0<<<grid(nblk), tpb, 0, s>>>(w, nblk, y); break;
        case QMM_TYPE_Q8_0:   k_deq_q8_0<<<grid(nblk), tpb, 0, s>>>(w, nblk, y); break;
        case QMM_TYPE_Q4_K:   k_deq_q4_K<<<grid(nblk * 4), tpb, 0, s>>>(w, nblk, y); break;
        case QMM_TYPE_Q6_K:   k_deq_q6_K<<<grid(nblk * 8), tpb, 0, s>>>(w, nblk, y); break;
        case QMM_TYPE_IQ4_XS: k_deq_iq4_xs<<<grid(nblk * 8), tpb, 0, s>>>(w, nblk, y); break;
        case QMM_TYPE_Q5_K:   k_deq_q5_K<<<grid(nblk * 4), tpb, 0, s>>>(w, nblk, y); break;
        case QMM_TYPE_IQ4_NL: k_deq_iq4_nl<<<grid(nblk), tpb, 0, s>>>(w, nblk, y); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qmm
