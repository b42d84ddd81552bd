/*
 * qmm_oracle.c - TEST INFRASTRUCTURE ONLY (see qmm_oracle.h).
 *
 * CPU restatement of ggml's arithmetic for MUL_MAT / MUL_MAT_ID on Q4_0,
 * Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL and IQ4_XS weights.  Each function names the reference
 * text it follows (paths relative to /root/reference; P01/P02/P03 =
 * contrib/llama.cpp/patches/0000-0{1,2,3}-*.patch).  Built with
 * -ffp-contract=off so that no multiply-add is fused behind our back.
 */
#include "qmm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

_Static_assert(sizeof(orc_block_q4_0) == 18, "block_q4_0");
_Static_assert(sizeof(orc_block_q8_0) == 34, "block_q8_0");
_Static_assert(sizeof(orc_block_q4_K) == 144, "block_q4_K");
_Static_assert(sizeof(orc_block_q6_K) == 210, "block_q6_K");
_Static_assert(sizeof(orc_block_iq4_xs) == 136, "block_iq4_xs");
_Static_assert(sizeof(orc_block_q5_K) == 176, "block_q5_K");
_Static_assert(sizeof(orc_block_iq4_nl) == 18, "block_iq4_nl");
_Static_assert(sizeof(orc_block_q8_K) == 292, "block_q8_K");

/* ---- IEEE binary16 <-> binary32 (from the IEEE 754 encoding) ------------ */

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_fp16_to_fp32(orc_half h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        const float v = (float)m * 5.9604644775390625e-8f;   /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* round to nearest, ties to even (what _cvtss_sh(x, 0) does on x86) */
orc_half orc_fp32_to_fp16(float f) {
    const uint32_t x = f32_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t e = (x >> 23) & 0xffu, m = x & 0x7fffffu;
    if (e == 0xff) return (orc_half)(sign | 0x7c00u | (m ? 0x200u : 0u));
    const int32_t he = (int32_t)e - 112;               /* exponent in half's bias */
    if (he >= 31) return (orc_half)(sign | 0x7c00u);
    if (he <= 0) {                                     /* half subnormal (or zero) */
        if (he < -10) return (orc_half)sign;
        const uint32_t mf = m | 0x800000u;
        const int shift = 14 - he;                     /* 14..24 */
        uint32_t hm = mf >> shift;
        const uint32_t rem = mf & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (orc_half)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)he << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;   /* a carry into the exponent is right */
    return (orc_half)h;
}

/* ---- type table (tools/coder_mtp_gguf.py:49-54) -------------------------- */

int orc_type_info(int type, int * blck, int * bytes, int * vec_dot_type) {
    int b = 0, s = 0, v = 0;
    switch (type) {
        case ORC_Q4_0:   b = 32;  s = 18;  v = ORC_Q8_0; break;
        case ORC_Q8_0:   b = 32;  s = 34;  v = ORC_Q8_0; break;
        case ORC_Q4_K:   b = 256; s = 144; v = ORC_Q8_K; break;
        case ORC_Q6_K:   b = 256; s = 210; v = ORC_Q8_K; break;
        case ORC_IQ4_XS: b = 256; s = 136; v = ORC_Q8_K; break;
        case ORC_Q5_K:   b = 256; s = 176; v = ORC_Q8_K; break;
        case ORC_IQ4_NL: b = 32;  s = 18;  v = ORC_Q8_0; break;
        case ORC_Q8_K:   b = 256; s = 292; v = 0; break;
        default: return 0;
    }
    if (blck) *blck = b;
    if (bytes) *bytes = s;
    if (vec_dot_type) *vec_dot_type = v;
    return 1;
}

/* the IQ4_NL / IQ4_XS non-linear codebook (P01:3335-3337) */
static const int8_t kvalues_iq4nl[16] = { -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113 };
const int8_t * orc_kvalues_iq4nl(void) { return kvalues_iq4nl; }

/* 6-bit scale and min j of a Q4_K super-block (P01:2164-2176, get_scale_min_k4) */
static void scale_min_k4(int j, const uint8_t * q, uint8_t * sc, uint8_t * m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m  = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m  = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ---- dequantize_row_* (a2; restated in tools/mtp_fit.py:360-409) -------- */

static void dequant_q4_0(const orc_block_q4_0 * x, float * y, int64_t nb) {
    for (int64_t i = 0; i < nb; ++i) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int j = 0; j < 16; ++j) {
            y[32 * i + j]      = (float)((x[i].qs[j] & 0xF) - 8) * d;   /* low nibbles: weights 0..15 */
            y[32 * i + j + 16] = (float)((x[i].qs[j] >> 4) - 8) * d;    /* high nibbles: 16..31 */
        }
    }
}

static void dequant_q8_0(const orc_block_q8_0 * x, float * y, int64_t nb) {
    for (int64_t i = 0; i < nb; ++i) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int j = 0; j < 32; ++j) y[32 * i + j] = (float)x[i].qs[j] * d;
    }
}

static void dequant_q4_K(const orc_block_q4_K * x, float * y, int64_t nb) {
    for (int64_t i = 0; i < nb; ++i) {
        const float d = orc_fp16_to_fp32(x[i].d), dmin = orc_fp16_to_fp32(x[i].dmin);
        const uint8_t * q = x[i].qs;
        float * out = y + 256 * i;
        for (int c = 0; c < 4; ++c) {               /* 64 weights from 32 bytes: low, then high nibbles */
            uint8_t sc, m;
            scale_min_k4(2 * c, x[i].scales, &sc, &m);
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            scale_min_k4(2 * c + 1, x[i].scales, &sc, &m);
            const float d2 = d * (float)sc, m2 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) out[64 * c + l]      = d1 * (float)(q[32 * c + l] & 0xF) - m1;
            for (int l = 0; l < 32; ++l) out[64 * c + 32 + l] = d2 * (float)(q[32 * c + l] >> 4) - m2;
        }
    }
}

/* 6-bit code of weight `w` (0..255) in a Q6_K super-block, 0..63 */
static int q6_code(const orc_block_q6_K * b, int w) {
    const int n = w / 128, r = w % 128, g = r / 32, l = r % 32;     /* half, quarter, position */
    const uint8_t ql = b->ql[64 * n + l + 32 * (g & 1)];
    const uint8_t qh = b->qh[32 * n + l];
    const int lo = (g < 2) ? (ql & 0xF) : (ql >> 4);
    return lo | (((qh >> (2 * g)) & 3) << 4);
}

static void dequant_q6_K(const orc_block_q6_K * x, float * y, int64_t nb) {
    for (int64_t i = 0; i < nb; ++i) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int w = 0; w < 256; ++w) {
            const int is = 8 * (w / 128) + 2 * ((w % 128) / 32) + (w % 32) / 16;   /* one scale per 16 */
            y[256 * i + w] = d * (float)x[i].scales[is] * (float)(q6_code(&x[i], w) - 32);
        }
    }
}

static int iq4xs_ls(const orc_block_iq4_xs * b, int ib) {
    return ((b->scales_l[ib / 2] >> (4 * (ib % 2))) & 0xF) | (((b->scales_h >> (2 * ib)) & 3) << 4);
}

static void dequant_iq4_xs(const orc_block_iq4_xs * x, float * y, int64_t nb) {
    for (int64_t i = 0; i < nb; ++i) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int ib = 0; ib < 8; ++ib) {
            const float dl = d * (float)(iq4xs_ls(&x[i], ib) - 32);
            const uint8_t * qs = x[i].qs + 16 * ib;
            for (int j = 0; j < 16; ++j) {
                y[256 * i + 32 * ib + j]      = dl * (float)kvalues_iq4nl[qs[j] & 0xF];
                y[256 * i + 32 * ib + j + 16] = dl * (float)kvalues_iq4nl[qs[j] >> 4];
            }
        }
    }
}

/* Q5_K: Q4_K's d, dmin and 6-bit scales/mins with a fifth code bit per weight.  Chunk c of 64
 * weights takes ql[32c + l] (low nibbles: weights 64c + l, high nibbles: 64c + 32 + l) and bits
 * 2c (low) / 2c + 1 (high) of qh[l] (ggml's dequantize_row_q5_K; the reference's decode of the
 * same fields, P01:3736-3750, mv_q45_K) */
static void dequant_q5_K(const orc_block_q5_K * x, float * y, int64_t nb) {
    for (int64_t i = 0; i < nb; ++i) {
        const float d = orc_fp16_to_fp32(x[i].d), dmin = orc_fp16_to_fp32(x[i].dmin);
        float * out = y + 256 * i;
        for (int c = 0; c < 4; ++c) {
            uint8_t sc, m;
            scale_min_k4(2 * c, x[i].scales, &sc, &m);
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            scale_min_k4(2 * c + 1, x[i].scales, &sc, &m);
            const float d2 = d * (float)sc, m2 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) {
                const uint8_t q = x[i].qs[32 * c + l], h = x[i].qh[l];
                out[64 * c + l]      = d1 * (float)((q & 0xF) + (((h >> (2 * c)) & 1) << 4)) - m1;
                out[64 * c + 32 + l] = d2 * (float)((q >> 4) + (((h >> (2 * c + 1)) & 1) << 4)) - m2;
            }
        }
    }
}

/* IQ4_NL: Q4_0's block (d, qs[16]) with the codes through the non-linear codebook instead of
 * q - 8 (ggml's dequantize_row_iq4_nl; the reference's mv_iq4_nl, P01:3414-3455) */
static void dequant_iq4_nl(const orc_block_iq4_nl * x, float * y, int64_t nb) {
    for (int64_t i = 0; i < nb; ++i) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int j = 0; j < 16; ++j) {
            y[32 * i + j]      = d * (float)kvalues_iq4nl[x[i].qs[j] & 0xF];
            y[32 * i + j + 16] = d * (float)kvalues_iq4nl[x[i].qs[j] >> 4];
        }
    }
}

void orc_dequantize_row(int type, const void * x, float * y, int64_t k) {
    int blck = 0;
    if (!orc_type_info(type, &blck, NULL, NULL)) return;
    const int64_t nb = k / blck;
    switch (type) {
        case ORC_Q4_0:   dequant_q4_0((const orc_block_q4_0 *)x, y, nb); break;
        case ORC_Q8_0:   dequant_q8_0((const orc_block_q8_0 *)x, y, nb); break;
        case ORC_Q4_K:   dequant_q4_K((const orc_block_q4_K *)x, y, nb); break;
        case ORC_Q6_K:   dequant_q6_K((const orc_block_q6_K *)x, y, nb); break;
        case ORC_IQ4_XS: dequant_iq4_xs((const orc_block_iq4_xs *)x, y, nb); break;
        case ORC_Q5_K:   dequant_q5_K((const orc_block_q5_K *)x, y, nb); break;
        case ORC_IQ4_NL: dequant_iq4_nl((const orc_block_iq4_nl *)x, y, nb); break;
        default: break;
    }
}

/* ---- activation quantizers (a3, a4) ------------------------------------ */

/* ggml-cpu's x86 quantize_row_q8_0 (P03:646-669): d = amax/127 stored as
 * fp16 (RNE); codes = round-half-even(x * (127/amax)), saturated to int8. */
void orc_quantize_row_q8_0(const float * x, void * vy, int64_t k) {
    orc_block_q8_0 * y = (orc_block_q8_0 *)vy;
    for (int64_t i = 0; i < k / 32; ++i, x += 32) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) { const float a = fabsf(x[j]); amax = a > amax ? a : amax; }
        y[i].d = orc_fp32_to_fp16(amax / 127.f);
        const float mul = amax != 0.0f ? 127.f / amax : 0.0f;
        for (int j = 0; j < 32; ++j) {
            float v = nearbyintf(x[j] * mul);            /* default rounding mode: ties to even */
            v = v > 127.f ? 127.f : (v < -128.f ? -128.f : v);
            y[i].qs[j] = (int8_t)v;
        }
    }
}

/* ggml's quantize_row_q8_K_ref (P03:673-683): mx = the first element of
 * largest |x|, iscale = -127/mx, codes = min(127, nearest(iscale*x)),
 * bsums = sums of 16 codes, d = 1/iscale; an all-zero block is all zero. */
void orc_quantize_row_q8_K(const float * x, void * vy, int64_t k) {
    orc_block_q8_K * y = (orc_block_q8_K *)vy;
    for (int64_t i = 0; i < k / 256; ++i, x += 256) {
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 256; ++j) {
            const float a = fabsf(x[j]);
            if (a > amax) { amax = a; mx = x[j]; }
        }
        if (amax == 0.0f) { memset(&y[i], 0, sizeof(y[i])); continue; }
        const float iscale = -127.f / mx;
        for (int j = 0; j < 256; ++j) {
            const int v = (int)nearbyintf(iscale * x[j]);
            y[i].qs[j] = (int8_t)(v > 127 ? 127 : v);
        }
        for (int j = 0; j < 16; ++j) {
            int s = 0;
            for (int l = 0; l < 16; ++l) s += y[i].qs[16 * j + l];
            y[i].bsums[j] = (int16_t)s;
        }
        y[i].d = 1.0f / iscale;
    }
}

void orc_quantize_act(int type, const float * x, void * y, int64_t k) {
    int vdt = 0;
    orc_type_info(type, NULL, NULL, &vdt);
    if (vdt == ORC_Q8_0) orc_quantize_row_q8_0(x, y, k);
    else orc_quantize_row_q8_K(x, y, k);
}

size_t orc_act_row_size(int type, int64_t k) {
    int vdt = 0;
    orc_type_info(type, NULL, NULL, &vdt);
    return vdt == ORC_Q8_0 ? (size_t)(k / 32) * sizeof(orc_block_q8_0) : (size_t)(k / 256) * sizeof(orc_block_q8_K);
}

/* ---- vec_dot closed forms (a5, a6) --------------------------------------
 * The integer sums are exact; the float combine is one fp32 accumulator per
 * row, block after block (ggml's generic order up to the lane split). */

static float dot_q4_0(int64_t nb, const orc_block_q4_0 * x, const orc_block_q8_0 * y) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; ++i) {
        int sumi = 0;
        for (int j = 0; j < 16; ++j) {
            sumi += ((x[i].qs[j] & 0xF) - 8) * y[i].qs[j];
            sumi += ((x[i].qs[j] >> 4) - 8) * y[i].qs[j + 16];
        }
        sumf += (float)sumi * (orc_fp16_to_fp32(x[i].d) * orc_fp16_to_fp32(y[i].d));
    }
    return sumf;
}

static float dot_q8_0(int64_t nb, const orc_block_q8_0 * x, const orc_block_q8_0 * y) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; ++i) {
        int sumi = 0;
        for (int j = 0; j < 32; ++j) sumi += x[i].qs[j] * y[i].qs[j];
        sumf += (float)sumi * (orc_fp16_to_fp32(x[i].d) * orc_fp16_to_fp32(y[i].d));
    }
    return sumf;
}

/* d_x * (fp16(d) * sum_j sc_j * sum_{l in j} q_l y_l - fp16(dmin) * sum_j m_j * bsum32_j) */
static float dot_q4_K(int64_t nb, const orc_block_q4_K * x, const orc_block_q8_K * y) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; ++i) {
        int sum_sc = 0, sum_m = 0;
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, m;
            scale_min_k4(j, x[i].scales, &sc, &m);
            const uint8_t * q = x[i].qs + 32 * (j / 2);
            const int8_t * a = y[i].qs + 32 * j;
            const int shift = 4 * (j & 1);
            int s = 0;
            for (int l = 0; l < 32; ++l) s += ((q[l] >> shift) & 0xF) * a[l];
            sum_sc += sc * s;
            sum_m += m * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        }
        const float d = orc_fp16_to_fp32(x[i].d) * y[i].d, dmin = orc_fp16_to_fp32(x[i].dmin) * y[i].d;
        sumf += d * (float)sum_sc;
        sumf -= dmin * (float)sum_m;
    }
    return sumf;
}

static float dot_q6_K(int64_t nb, const orc_block_q6_K * x, const orc_block_q8_K * y) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; ++i) {
        int sumi = 0;
        for (int is = 0; is < 16; ++is) {
            int s = 0;
            for (int l = 0; l < 16; ++l) {
                /* weight w of scale group `is`: half n, quarter g, position */
                const int n = is / 8, g = (is % 8) / 2, l0 = 16 * (is % 2) + l;
                const int w = 128 * n + 32 * g + l0;
                s += (q6_code(&x[i], w) - 32) * y[i].qs[w];
            }
            sumi += x[i].scales[is] * s;
        }
        sumf += (orc_fp16_to_fp32(x[i].d) * y[i].d) * (float)sumi;
    }
    return sumf;
}

static float dot_iq4_xs(int64_t nb, const orc_block_iq4_xs * x, const orc_block_q8_K * y) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; ++i) {
        const float d4d8 = orc_fp16_to_fp32(x[i].d) * y[i].d;
        for (int ib = 0; ib < 8; ++ib) {
            const uint8_t * qs = x[i].qs + 16 * ib;
            const int8_t * a = y[i].qs + 32 * ib;
            int s = 0;
            for (int j = 0; j < 16; ++j) {
                s += kvalues_iq4nl[qs[j] & 0xF] * a[j];
                s += kvalues_iq4nl[qs[j] >> 4] * a[j + 16];
            }
            sumf += (d4d8 * (float)(iq4xs_ls(&x[i], ib) - 32)) * (float)s;
        }
    }
    return sumf;
}

/* Q4_K's combine with 5-bit codes (ggml's vec_dot_q5_K_q8_K, generic form) */
static float dot_q5_K(int64_t nb, const orc_block_q5_K * x, const orc_block_q8_K * y) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; ++i) {
        int sum_sc = 0, sum_m = 0;
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, m;
            scale_min_k4(j, x[i].scales, &sc, &m);
            const uint8_t * q = x[i].qs + 32 * (j / 2);
            const int8_t * a = y[i].qs + 32 * j;
            const int shift = 4 * (j & 1);
            int s = 0;
            for (int l = 0; l < 32; ++l) s += (((q[l] >> shift) & 0xF) | (((x[i].qh[l] >> j) & 1) << 4)) * a[l];
            sum_sc += sc * s;
            sum_m += m * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        }
        const float d = orc_fp16_to_fp32(x[i].d) * y[i].d, dmin = orc_fp16_to_fp32(x[i].dmin) * y[i].d;
        sumf += d * (float)sum_sc;
        sumf -= dmin * (float)sum_m;
    }
    return sumf;
}

/* Q4_0's combine with codebook values (ggml's vec_dot_iq4_nl_q8_0) */
static float dot_iq4_nl(int64_t nb, const orc_block_iq4_nl * x, const orc_block_q8_0 * y) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; ++i) {
        int sumi = 0;
        for (int j = 0; j < 16; ++j) {
            sumi += kvalues_iq4nl[x[i].qs[j] & 0xF] * y[i].qs[j];
            sumi += kvalues_iq4nl[x[i].qs[j] >> 4] * y[i].qs[j + 16];
        }
        sumf += (orc_fp16_to_fp32(y[i].d) * orc_fp16_to_fp32(x[i].d)) * (float)sumi;
    }
    return sumf;
}

float orc_vec_dot(int type, int64_t k, const void * w, const void * xq) {
    switch (type) {
        case ORC_Q4_0:   return dot_q4_0(k / 32, (const orc_block_q4_0 *)w, (const orc_block_q8_0 *)xq);
        case ORC_Q8_0:   return dot_q8_0(k / 32, (const orc_block_q8_0 *)w, (const orc_block_q8_0 *)xq);
        case ORC_Q4_K:   return dot_q4_K(k / 256, (const orc_block_q4_K *)w, (const orc_block_q8_K *)xq);
        case ORC_Q6_K:   return dot_q6_K(k / 256, (const orc_block_q6_K *)w, (const orc_block_q8_K *)xq);
        case ORC_IQ4_XS: return dot_iq4_xs(k / 256, (const orc_block_iq4_xs *)w, (const orc_block_q8_K *)xq);
        case ORC_Q5_K:   return dot_q5_K(k / 256, (const orc_block_q5_K *)w, (const orc_block_q8_K *)xq);
        case ORC_IQ4_NL: return dot_iq4_nl(k / 32, (const orc_block_iq4_nl *)w, (const orc_block_q8_0 *)xq);
        default: return NAN;
    }
}

/* ---- drivers (a7): quantize src1 once, vec_dot per (row, column) --------- */

typedef struct {
    int type;
    const uint8_t * w;        /* expert 0, row 0 */
    size_t row_bytes;
    int64_t M, K;
    /* pairs: column xq[p], weight matrix wsel[p] (expert), output out[p] */
    const uint8_t * const * xq;
    const int64_t * wsel;
    float * const * out;
    int64_t npairs;
    int64_t r0, r1;           /* row range of this worker */
} orc_job;

static void * orc_worker(void * arg) {
    const orc_job * j = (const orc_job *)arg;
    for (int64_t p = 0; p < j->npairs; ++p) {
        if (j->wsel[p] < 0) continue;
        const uint8_t * wm = j->w + (size_t)j->wsel[p] * (size_t)j->M * j->row_bytes;
        for (int64_t r = j->r0; r < j->r1; ++r)
            j->out[p][r] = orc_vec_dot(j->type, j->K, wm + (size_t)r * j->row_bytes, j->xq[p]);
    }
    return NULL;
}

static void orc_run(int type, const void * w, int64_t M, int64_t K, const uint8_t * const * xq,
                    const int64_t * wsel, float * const * out, int64_t npairs, int nthreads) {
    int bytes = 0, blck = 1;
    orc_type_info(type, &blck, &bytes, NULL);
    if (nthreads <= 0) nthreads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (nthreads < 1) nthreads = 1;
    if (nthreads > M) nthreads = (int)M;
    orc_job * jobs = (orc_job *)calloc((size_t)nthreads, sizeof(orc_job));
    pthread_t * th = (pthread_t *)calloc((size_t)nthreads, sizeof(pthread_t));
    const int64_t per = (M + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; ++t) {
        orc_job * j = &jobs[t];
        j->type = type; j->w = (const uint8_t *)w; j->row_bytes = (size_t)(K / blck) * bytes;
        j->M = M; j->K = K; j->xq = xq; j->wsel = wsel; j->out = out; j->npairs = npairs;
        j->r0 = t * per; j->r1 = (t + 1) * per < M ? (t + 1) * per : M;
    }
    for (int t = 1; t < nthreads; ++t) pthread_create(&th[t], NULL, orc_worker, &jobs[t]);
    orc_worker(&jobs[0]);
    for (int t = 1; t < nthreads; ++t) pthread_join(th[t], NULL);
    free(jobs);
    free(th);
}

void orc_mul_mat(int type, const void * w, int64_t M, int64_t K, const float * x, int64_t N,
                 float * dst, int nthreads) {
    const size_t arow = orc_act_row_size(type, K);
    uint8_t * xq = (uint8_t *)malloc(arow * (size_t)N);
    const uint8_t ** cols = (const uint8_t **)malloc(sizeof(*cols) * (size_t)N);
    int64_t * wsel = (int64_t *)calloc((size_t)N, sizeof(int64_t));
    float ** out = (float **)malloc(sizeof(*out) * (size_t)N);
    for (int64_t n = 0; n < N; ++n) {
        orc_quantize_act(type, x + n * K, xq + n * arow, K);
        cols[n] = xq + n * arow;
        out[n] = dst + n * M;
    }
    orc_run(type, w, M, K, cols, wsel, out, N, nthreads);
    free(xq); free(cols); free(wsel); free(out);
}

/* MUL_MAT_ID (P01:3916-3922): pair (slot i, token t) uses expert ids[t][i],
 * column (i % ne11) of token t and writes dst[t][i]; a negative id writes
 * zeros (P02:98-103). */
void orc_mul_mat_id(int type, const void * w, int64_t M, int64_t K, int64_t E, const float * x,
                    int64_t ne11, const int32_t * ids, int64_t n_used, int64_t T, float * dst, int nthreads) {
    const size_t arow = orc_act_row_size(type, K);
    const int64_t ncols = ne11 * T, npairs = n_used * T;
    uint8_t * xq = (uint8_t *)malloc(arow * (size_t)ncols);
    for (int64_t c = 0; c < ncols; ++c) orc_quantize_act(type, x + c * K, xq + c * arow, K);
    const uint8_t ** cols = (const uint8_t **)malloc(sizeof(*cols) * (size_t)npairs);
    int64_t * wsel = (int64_t *)malloc(sizeof(int64_t) * (size_t)npairs);
    float ** out = (float **)malloc(sizeof(*out) * (size_t)npairs);
    for (int64_t t = 0; t < T; ++t) {
        for (int64_t i = 0; i < n_used; ++i) {
            const int64_t p = t * n_used + i;
            const int32_t e = ids[t * n_used + i];
            cols[p] = xq + (size_t)((i % ne11) + t * ne11) * arow;
            wsel[p] = (e >= 0 && e < E) ? e : -1;
            out[p] = dst + p * M;
            if (wsel[p] < 0) memset(out[p], 0, sizeof(float) * (size_t)M);
        }
    }
    orc_run(type, w, M, K, cols, wsel, out, npairs, nthreads);
    free(xq); free(cols); free(wsel); free(out);
}
