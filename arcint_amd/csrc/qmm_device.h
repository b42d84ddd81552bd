// qmm_device.h - device helpers for the gfx950 kernels of libqmm.
#pragma once

#include "qmm_internal.h"

namespace qmm {

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xffffu));
}

// v_dot4_i32_i8: c + sum of the four signed byte products
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// v_perm_b32: byte i of the result is byte sel.i of the 8-byte value
// {hi:lo} (lo supplies bytes 0-3, hi bytes 4-7)
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// the IQ4_NL / IQ4_XS codebook, four bytes per dword
constexpr int8_t kKvalues[16] = { -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113 };
constexpr uint32_t kv_word(int i) {
    return (uint32_t)(uint8_t)kKvalues[4 * i] | ((uint32_t)(uint8_t)kKvalues[4 * i + 1] << 8) |
           ((uint32_t)(uint8_t)kKvalues[4 * i + 2] << 16) | ((uint32_t)(uint8_t)kKvalues[4 * i + 3] << 24);
}

// four 4-bit codes (one per byte, bits 0-3) -> four int8 codebook values
__device__ __forceinline__ uint32_t iq4_lookup(uint32_t nib) {
    const uint32_t idx = nib & 0x07070707u;
    const uint32_t lo = perm(kv_word(1), kv_word(0), idx);   // entries 0..7
    const uint32_t hi = perm(kv_word(3), kv_word(2), idx);   // entries 8..15
    // byte i from lo (selector i) or hi (selector i + 4) by bit 3 of the code
    const uint32_t sel = ((nib >> 1) & 0x04040404u) | 0x03020100u;
    return perm(hi, lo, sel);
}

template <typename T>
__device__ __forceinline__ T ldg_nt(const T * p) {
    return __builtin_nontemporal_load(p);
}

__device__ __forceinline__ uint4 ld16_nt(const uint8_t * p) {
    const uint4 * q = reinterpret_cast<const uint4 *>(p);
    uint4 r;
    r.x = __builtin_nontemporal_load(&q->x);
    r.y = __builtin_nontemporal_load(&q->y);
    r.z = __builtin_nontemporal_load(&q->z);
    r.w = __builtin_nontemporal_load(&q->w);
    return r;
}

__device__ __forceinline__ uint4 ld16(const void * p) { return *reinterpret_cast<const uint4 *>(p); }

// sum over groups of `width` consecutive lanes (width a power of two <= 64)
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

}  // namespace qmm

namespace qmm {

// ---------------------------------------------------------------------------
// Activation quantizers, shared by the stand-alone pre-pass (k_quant.hip) and
// the GEMV's fused in-LDS quantization, so both are bit-identical with
// ggml-cpu's from_float (see k_quant.hip for the exact forms).
// ---------------------------------------------------------------------------
#pragma clang fp contract(off)

// q8_0 over 8 lanes (4 values each) of one 32-weight block; lane-group
// aligned (lanes 8g..8g+7).  Returns this lane's four codes packed; *d and
// *s (block scale, block code sum) are valid in every lane of the group.
__device__ __forceinline__ uint32_t quant_q8_0_lane(const float v[4], float * d, int * s) {
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    for (int o = 1; o < 8; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const _Float16 dh = (_Float16)(amax / 127.f);
    const float mul = amax != 0.0f ? 127.f / amax : 0.0f;
    int q[4], sum = 0;
    for (int i = 0; i < 4; ++i) {
        float r = __builtin_rintf(v[i] * mul);
        r = fminf(fmaxf(r, -128.f), 127.f);
        q[i] = (int)r;
        sum += q[i];
    }
    for (int o = 1; o < 8; o <<= 1) sum += __shfl_xor(sum, o, 64);
    *d = (float)dh;
    *s = sum;
    return (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
           ((uint32_t)(q[3] & 0xff) << 24);
}

// q8_K over a whole wave (4 values per lane, lane-major) of one 256-weight
// super-block.  Returns this lane's codes; *d is the block scale (all lanes),
// *bsum the sum of lanes 4b..4b+3's codes (valid in every lane of the quad).
__device__ __forceinline__ uint32_t quant_q8_K_wave(const float v[4], int lane, float * d, int * bsum) {
    float ba = -1.0f;
    int bi = 0;
    for (int i = 0; i < 4; ++i) {
        const float av = fabsf(v[i]);
        if (av > ba) { ba = av; bi = 4 * lane + i; }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float oa = __shfl_xor(ba, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (oa > ba || (oa == ba && oi < bi)) { ba = oa; bi = oi; }
    }
    const float pick = (bi & 3) == 0 ? v[0] : (bi & 3) == 1 ? v[1] : (bi & 3) == 2 ? v[2] : v[3];
    const float mx = __shfl(pick, bi >> 2, 64);
    int q[4] = { 0, 0, 0, 0 };
    float dv = 0.0f;
    if (ba != 0.0f) {
        const float iscale = -127.f / mx;
        for (int i = 0; i < 4; ++i) {
            const int r = (int)__builtin_rintf(iscale * v[i]);
            q[i] = r > 127 ? 127 : r;
        }
        dv = 1.0f / iscale;
    }
    int s = q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    *d = dv;
    *bsum = s;
    return (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
           ((uint32_t)(q[3] & 0xff) << 24);
}

#pragma clang fp contract(fast)

// f32 column c of an activation tensor (columns (i1, i2, i3), i1 fastest)
__device__ __forceinline__ const float * f32_col(const F32Cols & s, int64_t c) {
    const int64_t i1 = c % s.ne1, r = c / s.ne1, i2 = r % s.ne2, i3 = r / s.ne2;
    return reinterpret_cast<const float *>(s.base + i1 * s.nb1 + i2 * s.nb2 + i3 * s.nb3);
}

}  // namespace qmm
