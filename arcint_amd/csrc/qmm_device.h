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

// A constant in a VGPR.  gfx950's three-operand (VOP3) forms take no literal and read one SGPR
// at most, so with the codebook words and masks as literals each v_perm needs its table in
// registers anyway and each (x & m) | c becomes a v_and plus a v_or; with both in VGPRs the
// compiler fuses the pair into one v_and_or_b32.
template <int C>
__device__ __forceinline__ uint32_t in_vgpr() {
    uint32_t v;
    asm("v_mov_b32 %0, %1" : "=v"(v) : "i"(C));
    return v;
}

struct Iq4Regs { uint32_t k0, k1, k2, k3, m4, base; };

__device__ __forceinline__ Iq4Regs iq4_regs() {
    return { in_vgpr<(int)kv_word(0)>(), in_vgpr<(int)kv_word(1)>(), in_vgpr<(int)kv_word(2)>(),
             in_vgpr<(int)kv_word(3)>(), in_vgpr<0x04040404>(), in_vgpr<0x03020100>() };
}

// the eight 4-bit codes of q (both nibbles of its four bytes) -> their codebook values, lo from
// the low nibbles and hi from the high ones, iq4_lookup's three v_perm each, the selectors'
// shift shared and their mask-and-offset one v_and_or_b32: 13 VALU for the eight against 15-16
__device__ __forceinline__ void iq4_lookup8(uint32_t q, const Iq4Regs & k, uint32_t & lo, uint32_t & hi) {
    const uint32_t t = q >> 4;
    const uint32_t il = q & 0x07070707u, ih = t & 0x07070707u;
    const uint32_t sl = ((q >> 1) & k.m4) | k.base, sh = ((t >> 1) & k.m4) | k.base;
    lo = perm(perm(k.k3, k.k2, il), perm(k.k1, k.k0, il), sl);
    hi = perm(perm(k.k3, k.k2, ih), perm(k.k1, k.k0, ih), sh);
}

// iq4_lookup with the constants in VGPRs: the codes in bits 0-3 of each byte of x, bits 4-7
// ignored (x may be a byte-wise unmasked shift of the packed codes)
__device__ __forceinline__ uint32_t iq4_lookup_r(uint32_t x, const Iq4Regs & k) {
    const uint32_t il = x & 0x07070707u, sl = ((x >> 1) & k.m4) | k.base;
    return perm(perm(k.k3, k.k2, il), perm(k.k1, k.k0, il), sl);
}

// The GLU activations of ggml's split GLU (ggml-cpu vec.h scalar forms), fp32 with the device
// library's expf / tanhf / erff; glu_apply(op, x, g) = act(x) * g, REGLU as x > 0 ? x g : 0
__device__ __forceinline__ float glu_act(int op, float x) {
    switch (op) {
        case QMM_GLU_REGLU: return x > 0.0f ? x : 0.0f;
        case QMM_GLU_GEGLU: {
            const float k0 = 0.79788456080286535587989211986876f, k1 = 0.044715f;
            return 0.5f * x * (1.0f + tanhf(k0 * x * (1.0f + k1 * x * x)));
        }
        case QMM_GLU_SWIGLU: return x / (1.0f + expf(-x));
        case QMM_GLU_GEGLU_ERF: return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440084436210484f));
        case QMM_GLU_GEGLU_QUICK: return x * (1.0f / (1.0f + expf(-1.702f * x)));
        default: return 0.0f;
    }
}

__device__ __forceinline__ float glu_apply(int op, float x, float g) {
    return op == QMM_GLU_REGLU ? (x > 0.0f ? x * g : 0.0f) : glu_act(op, x) * g;
}

// four 4-bit codes 0..15 (one per byte) -> q - 8 as int8 (no borrow between bytes)
__device__ __forceinline__ uint32_t q4_minus8(uint32_t nib) {
    return (((nib | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
}

// four bytes times s with a packed 16-bit multiply; every product must be < 256 (no carries)
__device__ __forceinline__ uint32_t v2_mul(uint32_t v, uint32_t s) {
    typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
    const v2u16 a = __builtin_bit_cast(v2u16, v);
    const v2u16 b = { (unsigned short)s, (unsigned short)s };
    return __builtin_bit_cast(uint32_t, a * b);
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

// v + the value of lane sel(lane) of the same DPP row, by a DPP move
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    const int o = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false);
    return v + __builtin_bit_cast(float, o);
}

// Sum over groups of 2^log2w consecutive lanes (log2w <= 6); every lane of a
// group receives the group's sum.  Within a 16-lane DPP row the butterfly
// uses DPP moves (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror: each pairs every lane with one of the other half of its group
// of 2, 4, 8, 16); across rows it uses cross-lane permutes.
__device__ __forceinline__ float group_sum(float v, int log2w) {
    if (log2w >= 1) v = dpp_add<0xB1>(v);
    if (log2w >= 2) v = dpp_add<0x4E>(v);
    if (log2w >= 3) v = dpp_add<0x141>(v);
    if (log2w >= 4) v = dpp_add<0x140>(v);
    if (log2w >= 5) v += __shfl_xor(v, 16, 64);
    if (log2w >= 6) v += __shfl_xor(v, 32, 64);
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

// DPP lane moves used by the reductions below (all within one 16-lane row):
// 0xB1 quad_perm [1,0,3,2] (lane ^ 1), 0x4E quad_perm [2,3,0,1] (lane ^ 2),
// 0x141 row_half_mirror (lane i <-> 7 - i in each half row), 0x140
// row_mirror (i <-> 15 - i).  After the ^1 and ^2 steps every lane holds its
// quad's value, so a mirror step combines it with the other quad (half row)
// or the other half row.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) { return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v))); }

// max / sum over the 8 lanes of an aligned group (every lane gets the result)
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    return fmaxf(v, dpp_f<0x141>(v));
}
__device__ __forceinline__ int sum8(int v) {
    v += dpp_i<0xB1>(v);
    v += dpp_i<0x4E>(v);
    return v + dpp_i<0x141>(v);
}
__device__ __forceinline__ int sum4(int v) {
    v += dpp_i<0xB1>(v);
    return v + dpp_i<0x4E>(v);
}
// max over the whole wave, uniform result (row reduction by DPP, then the
// four row results read into scalars)
__device__ __forceinline__ float wave_max(float v) {
    v = max8(v);
    v = fmaxf(v, dpp_f<0x140>(v));
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
// q8_0 over 8 lanes (4 values each) of one 32-weight block; lane-group
// aligned (lanes 8g..8g+7), all 64 lanes active.  Returns this lane's four
// codes packed; *d and *s (block scale, block code sum) are valid in every
// lane of the group.
__device__ __forceinline__ uint32_t quant_q8_0_lane(const float v[4], float * d, int * s) {
    const float amax = max8(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    const _Float16 dh = (_Float16)(amax / 127.f);
    const float mul = amax != 0.0f ? 127.f / amax : 0.0f;
    int q[4], sum = 0;
    for (int i = 0; i < 4; ++i) {
        float r = QMM_RED == 2 ? roundf(v[i] * mul) : __builtin_rintf(v[i] * mul);   // (mutation 2: ties away)
        r = fminf(fmaxf(r, -128.f), 127.f);
        q[i] = (int)r;
        sum += q[i];
    }
    *d = (float)dh;
    *s = sum8(sum);
    return (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
           ((uint32_t)(q[3] & 0xff) << 24);
}

// q8_K over a whole wave (4 values per lane, element 4 * lane + i) of one
// 256-weight super-block, all 64 lanes active.  mx is the first element of
// largest |x|: the wave max of |x|, then the lowest lane holding it (ballot)
// and that lane's first such element.  Returns this lane's codes; *d is the
// block scale (all lanes), *bsum the sum of lanes 4b..4b+3's codes (valid in
// every lane of the quad).
__device__ __forceinline__ uint32_t quant_q8_K_wave(const float v[4], int lane, float * d, int * bsum) {
    (void)lane;
    const float a0 = fabsf(v[0]), a1 = fabsf(v[1]), a2 = fabsf(v[2]), a3 = fabsf(v[3]);
    const float amax = wave_max(fmaxf(fmaxf(a0, a1), fmaxf(a2, a3)));
    const float first = a0 == amax ? v[0] : a1 == amax ? v[1] : a2 == amax ? v[2] : v[3];
    const bool hit = a0 == amax || a1 == amax || a2 == amax || a3 == amax;
    const uint64_t mask = __ballot(hit);
    const int src = mask ? __builtin_ctzll(mask) : 0;
    const float mx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, first), src));
    int q[4] = { 0, 0, 0, 0 };
    float dv = 0.0f;
    if (amax != 0.0f) {
        const float iscale = -127.f / mx;
        for (int i = 0; i < 4; ++i) {
            const int r = (int)__builtin_rintf(iscale * v[i]);
            q[i] = r > 127 ? 127 : r;
        }
        dv = 1.0f / iscale;
    }
    *d = dv;
    *bsum = sum4(q[0] + q[1] + q[2] + q[3]);
    return (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
           ((uint32_t)(q[3] & 0xff) << 24);
}

#pragma clang fp contract(fast)

// f32 column c of an activation tensor (columns (i1, i2, i3), i1 fastest);
// column counts fit 32 bits, so the index split uses 32-bit divisions
__device__ __forceinline__ const float * f32_col(const F32Cols & s, int64_t c) {
    const uint32_t cc = (uint32_t)c, n1 = (uint32_t)s.ne1, n2 = (uint32_t)s.ne2;
    const uint32_t r = cc / n1, i1 = cc - r * n1, i3 = r / n2, i2 = r - i3 * n2;
    return reinterpret_cast<const float *>(s.base + (size_t)i1 * s.nb1 + (size_t)i2 * s.nb2 + (size_t)i3 * s.nb3);
}

// Activation quantization bodies, shared by the quantization launch and the
// MoE launch that also routes.  t = the thread's index over the quantization
// threads (whole waves; a block of threads is a multiple of 64).
#pragma clang fp contract(off)

// a / b (and a % b in r) for a, b >= 0: 32-bit when both fit, as they do for every realistic
// shape (a 64-bit division is a long instruction sequence ahead of a latency-bound kernel's
// first memory access)
__device__ __forceinline__ int64_t qdiv(int64_t a, int64_t b, int64_t & r) {
    if (((uint64_t)a | (uint64_t)b) < 0x80000000ull) {
        const uint32_t q = (uint32_t)a / (uint32_t)b;
        r = (int64_t)((uint32_t)a - q * (uint32_t)b);
        return (int64_t)q;
    }
    const int64_t q = a / b;
    r = a - q * b;
    return q;
}

// q8_0: 8 lanes per 32-weight block, 4 weights per lane
__device__ __forceinline__ void quant_q8_0_at(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, int64_t t) {
    const int64_t kq = a.ldk / 4;
    const bool live = t < ncols * kq;              // groups of 8 lanes are all live or all dead
    int64_t kr = 0;
    const int64_t c = live ? qdiv(t, kq, kr) : 0, k = live ? kr * 4 : 0;
    float v[4] = { 0.f, 0.f, 0.f, 0.f };
    if (live && k < K) {
        const float * x = f32_col(src, c) + k;
        for (int i = 0; i < 4; ++i) v[i] = x[i];
    }
    float d;
    int s;
    const uint32_t packed = quant_q8_0_lane(v, &d, &s);
    if (!live) return;
    *reinterpret_cast<uint32_t *>(a.codes + c * a.ldk + k) = packed;
    if ((t & 7) == 0) {
        const int64_t b = c * (a.ldk / 32) + k / 32;
        a.d[b] = d;
        a.sums[b] = (int16_t)s;
        if (a.dT) a.dT[(k / 32) * a.ldT + c] = d;            // padding blocks: d = 0
    }
}

// q8_K: one wave per 256-weight super-block, 4 weights per lane
__device__ __forceinline__ void quant_q8_K_at(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, int64_t t) {
    const int64_t wave = t >> 6;
    const int lane = (int)(t & 63);
    const int64_t nsb = a.ldk / 256;
    if (wave >= ncols * nsb) return;               // whole waves only
    int64_t sb;
    const int64_t c = qdiv(wave, nsb, sb);
    float v[4] = { 0.f, 0.f, 0.f, 0.f };
    if (sb * 256 < K) {
        const float * x = f32_col(src, c) + sb * 256 + 4 * lane;
        for (int i = 0; i < 4; ++i) v[i] = x[i];
    }
    float d;
    int s;
    const uint32_t packed = quant_q8_K_wave(v, lane, &d, &s);
    *reinterpret_cast<uint32_t *>(a.codes + c * a.ldk + sb * 256 + 4 * lane) = packed;
    if ((lane & 3) == 0) a.sums[c * (a.ldk / 16) + sb * 16 + (lane >> 2)] = (int16_t)s;
    if (a.bsp) {                                   // sub-block sums (8 lanes = 32 codes) as 64 bh + bl
        const int s32 = s + __shfl_xor(s, 4, 64);
        if ((lane & 7) == 0) {
            int8_t * o = a.bsp + (sb * a.ldT + c) * 16 + (lane >> 3);
            o[0] = (int8_t)(s32 >> 6);
            o[8] = (int8_t)(s32 & 63);
        }
    }
    if (lane == 0) {
        a.d[c * nsb + sb] = d;
        if (a.dT) a.dT[sb * a.ldT + c] = d;
    }
}

#pragma clang fp contract(fast)


// ---- the MoE router of one token, run by one wave -----------------------------------------
// Role of the reference's fused router (kernel_topk_moe_softmax_norm, P09:899-1000), which
// replaces llama.cpp's gating chain SOFT_MAX, ARGSORT (desc), VIEW, GET_ROWS, SUM_ROWS, CLAMP,
// DIV (matched at P02:786-821); the selection here is a filter and a count, not repeated arg-max
// rounds.  Lane l holds the logits of the NPER consecutive experts [l NPER, (l + 1) NPER).  The
// order is the reference's: the float32 values e = exp(x - max) it ranks (P09:935-966), equal
// values to the lower expert, so two distinct logits whose float32 exp is equal tie (as ggml's
// SOFT_MAX -> ARGSORT ranks float32 probabilities):
//  1. each e becomes a 32-bit key, its bits + 1 (e >= 0, so the bits are in e's order; an exp
//     that underflows to 0 still ranks above the padding); padding gets key 0;
//  2. the filter: tau0 = the k-th largest of the 64 lanes' largest keys with its low 14 bits
//     cleared, found most-significant bit first (16 steps of one ballot).  The lanes holding the
//     k largest maxima hold k keys >= tau0, so every winner is >= tau0;
//  3. the candidates (keys >= tau0; usually a few more than k) go to LDS, each lane's at the
//     places a ballot per held key gives it;
//  4. each candidate counts the candidates ahead of it (larger key, or equal key and lower
//     expert): those with fewer than k ahead win, at that rank.
// Weights: exp(x - max) / sum over all experts (a wave sum), divided by the winners' sum, taken
// in rank order and clamped to [cmin, cmax].  Only the calling wave takes part (its LDS traffic
// is ordered by wave-scope fences, no work-group barrier): cand_key / cand_exp hold n_expert
// entries, ranked_p 32; the winners go to rid[r] (expert) and rw[r] (weight), r < k.

__device__ __forceinline__ float wave_sum_f(float v) {
    // rows by DPP (every lane of a row ends with the row's sum: a + b and b + a are the same
    // float), then the four row sums in a fixed order
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

// the wave's LDS writes before this are seen by its loads after it
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int NPER>
__device__ __forceinline__ void topk_wave(const float * x, int n_expert, int k, float cmin, float cmax, int lane,
                                          uint32_t * cand_key, int * cand_exp, float * ranked_p, int32_t * rid,
                                          float * rw) {
    const int e0 = lane * NPER;
    float v[NPER];
    uint32_t key[NPER];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
        v[j] = e0 + j < n_expert ? x[e0 + j] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    const float m = wave_max(mx);
    float part = 0.0f;
    uint32_t kmax = 0;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
        const bool live = e0 + j < n_expert;
        const float e = live ? expf(v[j] - m) : 0.0f;
        part += e;
        key[j] = live ? __builtin_bit_cast(uint32_t, e) + 1u : 0u;
        kmax = key[j] > kmax ? key[j] : kmax;
    }
    const float S = wave_sum_f(part);
    // 2. tau0: the largest value of the key's bits 29..14 (lower bits zero) with at least k lane
    // maxima at or above it (keys are <= bits(1.0f) + 1 < 2^30): the k-th largest lane maximum
    // with its low bits cleared, so every winner is still >= tau0
    uint32_t tau0 = 0;
#pragma unroll
    for (int b = 29; b >= 14; --b) {
        const uint32_t c = tau0 | (1u << b);
        if (__popcll(__ballot(kmax >= c)) >= k) tau0 = c;
    }
    // 3. the candidates into LDS: per j, a ballot gives each lane its place among the lanes
    // holding one (the order of the candidates does not matter to the ranking below)
    int ncand = 0;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
        const uint64_t m = __ballot(key[j] >= tau0);
        if (key[j] >= tau0) {
            const int slot = ncand + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
            cand_key[slot] = key[j];
            cand_exp[slot] = e0 + j;
        }
        ncand += __popcll(m);
    }
    wave_lds_sync();
    // 4. each candidate's rank; the first k are the winners (their probabilities summed in
    // rank order).  A winner's probability is its e / S: e is its key less one, as bits.
    if (ncand <= 64) {                                            // uniform: one candidate per lane
        // (the candidates broadcast from registers by readlane: no LDS round trip per compare)
        const uint32_t ck = lane < ncand ? cand_key[lane] : 0u;
        const int ce = lane < ncand ? cand_exp[lane] : 0;
        int r = 0;
        for (int i = 0; i < ncand; ++i) {                         // uniform
            const uint32_t ki = (uint32_t)__builtin_amdgcn_readlane((int)ck, i);
            const int ei = __builtin_amdgcn_readlane(ce, i);
            r += ki > ck || (ki == ck && ei < ce);
        }
        const bool win = lane < ncand && r < k;
        const float pr = win ? __builtin_bit_cast(float, ck - 1u) / S : 0.0f;
        float wsum = 0.0f;
        for (int i = 0; i < k; ++i) {                             // uniform, in rank order
            const uint64_t at = __ballot(win && r == i);
            wsum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pr),
                                                                        at ? (int)__builtin_ctzll(at) : 0));
        }
        const float cl = fminf(fmaxf(wsum, cmin), cmax);
        if (win) {
            rid[r] = ce;
            rw[r] = pr / cl;
        }
        return;
    }
    constexpr int kMaxMine = 1024 / 64;
    int my_rank[kMaxMine], my_exp[kMaxMine];
    float my_p[kMaxMine];
    int nmine = 0;
    for (int c = lane; c < ncand; c += 64) {
        const uint32_t ku = cand_key[c];
        const int ke = cand_exp[c];
        int r = 0;
        for (int i = 0; i < ncand && r < k; ++i) r += cand_key[i] > ku || (cand_key[i] == ku && cand_exp[i] < ke);
        if (r < k) {
            const float p = __builtin_bit_cast(float, ku - 1u) / S;
            ranked_p[r] = p;
            my_rank[nmine] = r;
            my_exp[nmine] = ke;
            my_p[nmine] = p;
            ++nmine;
        }
    }
    wave_lds_sync();
    float wsum = 0.0f;
    for (int i = 0; i < k; ++i) wsum += ranked_p[i];               // uniform, in rank order
    const float cl = fminf(fmaxf(wsum, cmin), cmax);
    for (int q = 0; q < nmine; ++q) {
        rid[my_rank[q]] = my_exp[q];
        rw[my_rank[q]] = my_p[q] / cl;
    }
}

// topk_wave for any n_expert <= 1024 (lanes hold ceil(n_expert / 64) rounded up to a power of 2)
__device__ __forceinline__ void topk_wave_any(const float * x, int n_expert, int k, float cmin, float cmax, int lane,
                                              uint32_t * cand_key, int * cand_exp, float * ranked_p, int32_t * rid,
                                              float * rw) {
    const int nper = (n_expert + 63) / 64;
    if (nper <= 1) topk_wave<1>(x, n_expert, k, cmin, cmax, lane, cand_key, cand_exp, ranked_p, rid, rw);
    else if (nper <= 2) topk_wave<2>(x, n_expert, k, cmin, cmax, lane, cand_key, cand_exp, ranked_p, rid, rw);
    else if (nper <= 4) topk_wave<4>(x, n_expert, k, cmin, cmax, lane, cand_key, cand_exp, ranked_p, rid, rw);
    else if (nper <= 8) topk_wave<8>(x, n_expert, k, cmin, cmax, lane, cand_key, cand_exp, ranked_p, rid, rw);
    else topk_wave<16>(x, n_expert, k, cmin, cmax, lane, cand_key, cand_exp, ranked_p, rid, rw);
}

}  // namespace qmm
