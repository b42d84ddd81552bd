/*
 * qmm_oracle.h - TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of ggml's CPU arithmetic for the quantized matrix
 * product (ggml @ llama.cpp 3e4dfa8f39f904e681737d9f512a6e6338d848aa, which
 * arcint pins at contrib/packaging/arcint/build-deb.sh:31-33 and which is not
 * vendored in the reference).  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline; the product (libqmm) never calls it.
 *
 * What pins each part (the tests under tests/test_oracle*.py):
 *   dequantize_row_*      closed forms on hand-built blocks, exhaustive
 *                         scale-byte unpack, the kvalues_iq4nl table,
 *                         exact-representability invariants
 *   quantize_row_q8_0     the x86 form restated at 0000-03-...patch:646-669:
 *                         all-equal blocks, ties, zero blocks, saturation
 *   quantize_row_q8_K     ggml's _ref form restated at 0000-03-...patch:673-683:
 *                         sign of the first max-|x|, bsums, zero blocks
 *   vec_dot_*             integer exactness and the textbook identity
 *                         dot == sum(dequant(w) * dequant(q8(x))) in fp64
 *   mul_mat / mul_mat_id  index semantics of P01:3916-3922 and P02:90-124
 * Parity unpinned: ggml-cpu's SIMD float-combine order (AVX2/AVX-512) and its
 * thread chunking; this file follows the generic scalar order.
 */
#ifndef QMM_ORACLE_H
#define QMM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK4_0 32
#define ORC_QK8_0 32
#define ORC_QK_K  256

typedef uint16_t orc_half;

/* ggml's block structs, byte for byte (ggml-common.h at the pin) */
typedef struct { orc_half d; uint8_t qs[ORC_QK4_0 / 2]; } orc_block_q4_0;                  /* 18  */
typedef struct { orc_half d; int8_t  qs[ORC_QK8_0]; } orc_block_q8_0;                      /* 34  */
typedef struct { orc_half d; orc_half dmin; uint8_t scales[12]; uint8_t qs[ORC_QK_K / 2]; } orc_block_q4_K; /* 144 */
typedef struct { uint8_t ql[ORC_QK_K / 2]; uint8_t qh[ORC_QK_K / 4]; int8_t scales[ORC_QK_K / 16]; orc_half d; } orc_block_q6_K; /* 210 */
typedef struct { orc_half d; uint16_t scales_h; uint8_t scales_l[ORC_QK_K / 64]; uint8_t qs[ORC_QK_K / 2]; } orc_block_iq4_xs; /* 136 */
typedef struct { orc_half d; orc_half dmin; uint8_t scales[12]; uint8_t qh[ORC_QK_K / 8]; uint8_t qs[ORC_QK_K / 2]; } orc_block_q5_K; /* 176 */
typedef struct { orc_half d; uint8_t qs[ORC_QK4_0 / 2]; } orc_block_iq4_nl;                /* 18  */
typedef struct { float d; int8_t qs[ORC_QK_K]; int16_t bsums[ORC_QK_K / 16]; } orc_block_q8_K; /* 292 */

/* type ids as ggml_type */
enum { ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_Q8_K = 15, ORC_IQ4_NL = 20,
       ORC_IQ4_XS = 23 };

float    orc_fp16_to_fp32(orc_half h);
orc_half orc_fp32_to_fp16(float f);          /* round to nearest even, like F16C imm 0 */
int      orc_type_info(int type, int * blck, int * bytes, int * vec_dot_type);
const int8_t * orc_kvalues_iq4nl(void);

void orc_dequantize_row(int type, const void * x, float * y, int64_t k);
void orc_quantize_row_q8_0(const float * x, void * y, int64_t k);
void orc_quantize_row_q8_K(const float * x, void * y, int64_t k);
/* from_float of the vec_dot type of `type` (q8_0 for Q4_0/Q8_0/IQ4_NL, q8_K else) */
void orc_quantize_act(int type, const float * x, void * y, int64_t k);
size_t orc_act_row_size(int type, int64_t k);

/* one row of weights against one quantized activation row */
float orc_vec_dot(int type, int64_t k, const void * w, const void * xq);

/* dst[n*M + m] = sum_k W[m][k] * x[n*K + k]; W rows are GGUF blocks.
 * The activations are quantized first, once per column, as ggml-cpu does. */
void orc_mul_mat(int type, const void * w, int64_t M, int64_t K, const float * x, int64_t N,
                 float * dst, int nthreads);
/* experts w [E][M] rows; x [T][ne11][K]; ids [T][n_used]; dst [T][n_used][M] */
void orc_mul_mat_id(int type, const void * w, int64_t M, int64_t K, int64_t E, const float * x,
                    int64_t ne11, const int32_t * ids, int64_t n_used, int64_t T, float * dst, int nthreads);

#ifdef __cplusplus
}
#endif

#endif
