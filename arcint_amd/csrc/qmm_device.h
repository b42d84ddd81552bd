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
