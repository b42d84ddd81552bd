// qmm_internal.h - layouts and launch interfaces shared by the libqmm host
// code and its HIP kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/qmm.h"

namespace qmm {

// ---------------------------------------------------------------------------
// Weight layout in HBM.
//
// A quantized tensor of nblk GGUF blocks is stored as up to four planes, one
// per block field, each plane 256-byte aligned and holding that field of
// every block in block order (block i = row * blocks_per_row + kb, rows of
// all experts back to back).  The field split is chosen so that every plane
// a decode kernel streams is 16-byte aligned per block, which gives each lane
// 128-bit loads:
//   Q4_0   qs[16] | d[2]
//   Q8_0   qs[32] | d[2]
//   Q4_K   qs[128] | {d, dmin, scales[12]}[16]
//   Q6_K   ql[128] | qh[64] | scales[16] | d[2]
//   IQ4_XS qs[128] | {d, scales_h, scales_l[4]}[8]
// ---------------------------------------------------------------------------
struct Field { int off, size; };

struct TypeLayout {
    int type;
    int blck;       // weights per block
    int bytes;      // GGUF bytes per block
    int nfields;
    Field f[4];
};

const TypeLayout * type_layout(int type);   // nullptr for unknown types
size_t plane_bytes(const TypeLayout & L, int q, int64_t nblk);
size_t planes_alloc(const TypeLayout & L, int64_t nblk, size_t plane_off[4]);

constexpr size_t kPlaneAlign = 256;
static inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ---------------------------------------------------------------------------
// Quantized activations (the vec_dot type's from_float, done on the device).
// For column c of ncols:
//   codes  int8 [c][K]
//   d      f32  [c][K/bs]       bs = 32 (q8_0) or 256 (q8_K); q8_0's d is
//                               the fp16-rounded scale widened to f32
//   sums   i16  [c][K/ss]       ss = 32 (q8_0: sum of the block's codes)
//                               or 16 (q8_K: ggml's bsums)
// ---------------------------------------------------------------------------
struct ActBuf {
    int8_t *   codes;
    float *    d;
    int16_t *  sums;
    float *    dT;         // non-null: the scales again, block-major: dT[b * ldT + c]
    int64_t    ldT;        // >= ncols + 64 (the GEMM reads whole 64-column tiles)
    int64_t    K;
    int64_t    ncols;
    int        vdt;        // QMM_TYPE_Q8_0 or QMM_TYPE_Q8_K
};

__host__ __device__ static inline int act_block(int vdt) { return vdt == QMM_TYPE_Q8_0 ? 32 : 256; }
__host__ __device__ static inline int act_sum_block(int vdt) { return vdt == QMM_TYPE_Q8_0 ? 32 : 16; }
__host__ __device__ static inline int vec_dot_type(int type) {
    return (type == QMM_TYPE_Q4_0 || type == QMM_TYPE_Q8_0) ? QMM_TYPE_Q8_0 : QMM_TYPE_Q8_K;
}

// f32 source columns: column c = (i1, i2, i3) with i1 fastest
struct F32Cols {
    const char * base;
    int64_t ne1, ne2;          // to split c into (i1, i2, i3)
    size_t nb1, nb2, nb3;
};

// ---------------------------------------------------------------------------
// Weight views handed to kernels
// ---------------------------------------------------------------------------
struct WView {
    const uint8_t * p[4];      // planes
    int64_t bpr;               // blocks per row
    int64_t rows_per_mat;      // M (one expert / one 2-D slice)
};

// A GEMV task: up to 8 columns against one weight matrix.
constexpr int kMaxTaskCols = 8;
struct GemvTask {
    int32_t mat;                   // weight matrix (expert / slice) index; <0: skip
    int32_t ncols;
    int32_t col[kMaxTaskCols];     // activation column ids
    int64_t dst_off[kMaxTaskCols]; // float offset of dst row 0 for that column
};

// ---------------------------------------------------------------------------
// Launchers (defined in the .hip files); all enqueue on `s`.
// ---------------------------------------------------------------------------
hipError_t launch_dequant(int type, const WView & w, int64_t nblk, float * y, hipStream_t s);
hipError_t launch_quantize(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, hipStream_t s);
// writes ggml block bytes (block_q8_0 / block_q8_K) of an ActBuf into `out` (device)
hipError_t launch_act_to_blocks(const ActBuf & a, void * out, hipStream_t s);

// Dense MUL_MAT batch description (columns of one batch are contiguous ids)
struct GemvDense {
    int64_t ne11, ne12, ne13, r2, r3, ne02;
    int64_t d_nb1, d_nb2, d_nb3;   // dst strides in floats
};

// GEMV: dst[dst_off + m] for m < M, rows of matrix `mat` of each task.
// Activations come pre-quantized (`a`) or as f32 columns (`src`) that every
// work-group quantizes into LDS itself (bit-identical to the pre-pass).
// List mode (tasks != nullptr): `ntasks_dev` (optional) bounds the task list
// on the device, ntasks_max sizes the grid.  Dense mode (tasks == nullptr):
// tasks of up to nc columns are derived from `dense`.
hipError_t launch_gemv_any(int type, const WView & w, int64_t M, int64_t K, const ActBuf * a, const F32Cols * src,
                           const GemvTask * tasks, int ntasks_max, const int32_t * ntasks_dev, int nc,
                           const GemvDense * dense, float * dst, hipStream_t s);

// Prefill GEMM (int8 MFMA): for every batch b < nbatch, dst[doff(b) + n * d_nb1
// + m] = W(mat(b)) row m . activation column col0(b) + n, for n < N, m < M.
// Activations come from the pre-pass with block-major scales (a.dT).
struct GemmBatch {
    int64_t ne12, r2, r3, ne02;    // batch b = (i2, i3): mat = i2 / r2 + (i3 / r3) * ne02
    int64_t d_nb1, d_nb2, d_nb3;   // dst strides in floats
};
hipError_t launch_gemm(int type, const WView & w, int64_t M, int64_t K, const ActBuf & a, int64_t N, int64_t nbatch,
                       const GemmBatch & bt, float * dst, hipStream_t s);

// MoE routing: builds GEMV tasks (one per expert and up to 8 pairs) from ids.
struct RouteArgs {
    const int32_t * ids;        // [T][n_used] with row stride ids_nb1 (bytes)
    size_t ids_nb0, ids_nb1;
    int64_t n_used, T, ne11, n_as;
    int64_t dst_nb1, dst_nb2;   // float strides of dst dims 1 and 2
};
// scratch: counts [n_as], offsets [n_as], pairs [T*n_used]; tasks out
hipError_t launch_route(const RouteArgs & r, int32_t * scratch, GemvTask * tasks, int32_t * ntasks,
                        float * dst, int64_t M, hipStream_t s);

}  // namespace qmm
