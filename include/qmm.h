/*
 * qmm.h - C ABI of libqmm, an MI355X (gfx950) implementation of ggml's
 * quantized matrix product: GGML_OP_MUL_MAT and GGML_OP_MUL_MAT_ID on GGUF
 * block-quant weights (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS) with f32
 * activations.
 *
 * The entry points mirror what a ggml backend exposes for this op, so that a
 * ggml backend adaptor (or a ctypes harness) can bind them with plain
 * pointers and sizes.  Reference interfaces replaced, by entry point (paths
 * relative to the arcint tree; P01/P02 = contrib/llama.cpp/patches/
 * 0000-01-kquant-integer-dpas.patch / 0000-02-lowbit-iq-types.patch):
 *
 *   qmm_ctx_create/free          ggml_backend_opencl init / free; the device
 *                                context that owns the queue and scratch
 *                                (P01:43-60 prealloc_kq_* buffers)
 *   qmm_buffer_alloc/free        ggml_backend_buffer_type alloc_buffer / free
 *   qmm_tensor_alloc_size        buffer type get_alloc_size (planar layouts
 *                                need more than ggml_nbytes)
 *   qmm_tensor_set/get           buffer set_tensor / get_tensor: GGUF block
 *                                bytes in, device planes, exact bytes back
 *                                (P02:1556-1790)
 *   qmm_tensor_pack/unpack       the same GGUF <-> device-image conversion on
 *                                the host, for loaders that upload a prebuilt
 *                                image (the role of the planar-layout header
 *                                ggml-opencl-planes.h, 0116-...patch:17-159)
 *   qmm_supports_op              ggml_opencl_supports_op for MUL_MAT /
 *                                MUL_MAT_ID (P01:615-660)
 *   qmm_mul_mat                  ggml_cl_mul_mat (P01:1135-1160)
 *   qmm_mul_mat_id               ggml_cl_mul_mat_id (P01:1316-1325)
 *   qmm_mul_mat_noalloc          no counterpart in the reference: qmm_mul_mat for
 *                                callers that cannot allocate device memory
 *   qmm_graph_compute            ggml_backend_opencl_graph_compute over a node
 *                                list, graph_gen++ per call (P01:609-612);
 *                                activation dedup keyed per graph (P01:683-717)
 *   qmm_capture_begin/end,       no counterpart in the reference (OpenCL has no
 *   qmm_graph_launch/free        graph replay): HIP-graph capture and replay of
 *                                the ops on the context's stream, for decode
 *                                loops bound by launch latency
 *   qmm_dequantize               dequantize_row_* of ggml (bit-exact gate;
 *                                tools/mtp_fit.py:338-409 restates them;
 *                                Q5_K / IQ4_NL decode as P01:3736-3750 and
 *                                P01:3414-3455)
 *   qmm_quantize_act             ggml-cpu's from_float for the vec_dot type
 *                                (quantize_row_q8_0 / quantize_row_q8_K,
 *                                restated at 0000-03-...patch:646-683)
 *   qmm_synchronize              ggml_backend_synchronize (clFinish)
 *   qmm_last_error               the reason behind a failed status (the
 *                                reference aborts via GGML_ASSERT/CL_CHECK)
 *   qmm_downgrades               ggml_backend_opencl_downgrades() (0100-...patch:11-23)
 *   qmm_describe_mul_mat         the path and launch shape a MUL_MAT would take,
 *                                what GGML_OPENCL_FEWQ_LOG / _TRACE log per
 *                                shape (docs/switches.md:189-190)
 *   qmm_mul_mat_glu,             the reference's fuse_mm_glu chains (MUL_MAT /
 *   qmm_mul_mat_id_glu           MUL_MAT_ID gate and up, then GLU)
 *   qmm_moe_topk                 kernel_topk_moe_softmax_norm (P09:899-1000)
 *   qmm_moe_combine              the weights' MUL and the slot ADDs of
 *                                llama.cpp's build_moe_ffn
 *   qmm_moe_ffn                  no one call in the reference: the router,
 *                                expert products, GLU, down and combine of a
 *                                MoE FFN block (with a shared expert) in two
 *                                launches, for an adaptor that matches the chain
 *
 * Conventions (ggml's): a tensor is { type, ne[4], nb[4], data }.  For a
 * quantized type ne[0] is the row length in weights and must be a multiple
 * of the block size; nb[] are the strides of the GGUF byte layout.  The
 * device keeps quantized tensors in its own planar layout, so data of a
 * quantized tensor must be written and read through qmm_tensor_set/get.
 * The ops take a quantized view as src0 when the base image holds its rows
 * as whole matrices of the base (a slice of an expert stack; the reference's
 * whole-slice rule, 0116-opencl-q3_K.patch:76-85) or, when the base's
 * matrices are whole 64-row tiles, as whole tiles (a reshape [K, M*E] of
 * [K, M, E], rows 64i.. of a matrix); qmm_supports_op says no, with the
 * reason, for any other view.
 *   MUL_MAT:    src0 [K, M, ne02, ne03] quantized, src1 [K, N, ne12, ne13]
 *               f32, dst [M, N, ne12, ne13] f32; dst[m,n] = sum_k src0[k,m] *
 *               src1[k,n], src0 broadcast over dims 2 and 3 (ne12 % ne02 == 0).
 *   MUL_MAT_ID: src0 [K, M, n_as] quantized experts, src1 [K, ne11, T] f32
 *               with ne11 == 1 (broadcast) or ne11 == n_used, ids [n_used, T]
 *               i32, dst [M, n_used, T]; dst[:, i, t] = src0[:, :, ids[i,t]] *
 *               src1[:, i % ne11, t]; a negative id writes a zero row.
 * Threading: one in-order HIP stream per context; a context is not
 * thread-safe, like a ggml backend.
 */
#ifndef QMM_H
#define QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml_type ids (tools/coder_mtp_gguf.py:49-54) */
enum qmm_type {
    QMM_TYPE_F32    = 0,
    QMM_TYPE_F16    = 1,
    QMM_TYPE_Q4_0   = 2,
    QMM_TYPE_Q8_0   = 8,
    QMM_TYPE_Q4_K   = 12,
    QMM_TYPE_Q5_K   = 13,
    QMM_TYPE_Q6_K   = 14,
    QMM_TYPE_Q8_K   = 15,
    QMM_TYPE_IQ4_NL = 20,
    QMM_TYPE_IQ4_XS = 23,
    QMM_TYPE_I32    = 26,
};

/* ggml_op ids are not stable across ggml versions; the ABI uses its own */
enum qmm_op {
    QMM_OP_NONE       = 0,
    QMM_OP_MUL_MAT    = 1,
    QMM_OP_MUL_MAT_ID = 2,
};

/* GLU activations of qmm_mul_mat_glu: ggml's enum ggml_glu_op names (REGLU, GEGLU, SWIGLU,
 * GEGLU_ERF, GEGLU_QUICK; SWIGLU_OAI is not taken) with values of this ABI */
enum qmm_glu {
    QMM_GLU_REGLU       = 0,
    QMM_GLU_GEGLU       = 1,
    QMM_GLU_SWIGLU      = 2,
    QMM_GLU_GEGLU_ERF   = 4,
    QMM_GLU_GEGLU_QUICK = 5,
};

enum qmm_status {
    QMM_OK            = 0,
    QMM_ERR_INVALID   = 1,   /* shape / type / stride precondition */
    QMM_ERR_UNSUPPORTED = 2, /* qmm_supports_op would say no */
    QMM_ERR_DEVICE    = 3,   /* a HIP call failed */
    QMM_ERR_NOMEM     = 4,
};

typedef struct qmm_ctx    qmm_ctx;
typedef struct qmm_buffer qmm_buffer;

/* A non-owning view, like ggml_tensor: data lives at buffer + offs.
 * view_src / view_offs are ggml_tensor's own fields: the tensor whose
 * allocation this one views (never itself a view; NULL for a tensor that is
 * its own allocation) and the byte offset of this view's first byte in
 * view_src's GGUF layout.  A plain-typed (f32/f16/i32) tensor is addressed by
 * its buffer + offs whatever view_src says.  A quantized view reads and
 * writes its base's device image: its own buffer and offs are not used, and
 * byte b of the view is byte view_offs + b of the base (the reference's rule,
 * 0116-opencl-q3_K.patch:56-59 ggml_cl_lb_base and :113-133). */
typedef struct qmm_tensor {
    int32_t      type;   /* enum qmm_type */
    int64_t      ne[4];
    size_t       nb[4];  /* byte strides of the logical (GGUF) layout */
    qmm_buffer * buffer;
    size_t       offs;
    const struct qmm_tensor * view_src;
    size_t       view_offs;
} qmm_tensor;

/* One node of an op graph (ggml_tensor's op + src[0..2]). */
typedef struct qmm_node {
    int32_t      op;     /* enum qmm_op */
    qmm_tensor * src0;
    qmm_tensor * src1;
    qmm_tensor * ids;    /* MUL_MAT_ID only */
    qmm_tensor * dst;
} qmm_node;

/* ---- context and memory ------------------------------------------------ */
int    qmm_ctx_create(int device, qmm_ctx ** out);
void   qmm_ctx_free(qmm_ctx * ctx);
const char * qmm_last_error(qmm_ctx * ctx);  /* never NULL */

int    qmm_buffer_alloc(qmm_ctx * ctx, size_t size, qmm_buffer ** out);
void   qmm_buffer_free(qmm_ctx * ctx, qmm_buffer * buf);
size_t qmm_buffer_size(const qmm_buffer * buf);
/* device address of the buffer (for harnesses that share device memory) */
void * qmm_buffer_base(const qmm_buffer * buf);

/* bytes a contiguous tensor of this type and shape occupies on the device:
 * rows in tiles of 64, the K axis in groups of 256 weights, zero padding */
size_t qmm_tensor_alloc_size(int32_t type, const int64_t ne[4]);
/* bytes of the GGUF layout (ggml_nbytes of a contiguous tensor) */
size_t qmm_tensor_nbytes(int32_t type, const int64_t ne[4]);
/* block size (weights per block) and block bytes of a type; 0 if unknown */
int    qmm_type_block(int32_t type, size_t * block_bytes);

/* Write / read `size` bytes at byte `offset` of the tensor's GGUF layout
 * (ggml_backend_tensor_set/get: the range lies inside ggml_nbytes of the
 * tensor, strides notwithstanding).  Any byte range: a block that the range
 * covers in part is read, patched and written back.  A quantized view goes
 * through its base (view_src) at view_offs + offset, so every view of a
 * weight - permuted, reshaped, a slice or rows of it - moves the bytes the
 * base's layout puts there.  Both are synchronous with respect to the host
 * buffer. */
int    qmm_tensor_set(qmm_ctx * ctx, const qmm_tensor * t, const void * data, size_t offset, size_t size);
int    qmm_tensor_get(qmm_ctx * ctx, const qmm_tensor * t, void * data, size_t offset, size_t size);
/* Host only, no device: the device image (qmm_tensor_alloc_size bytes) of a
 * whole contiguous quantized tensor from its GGUF bytes, and back.  Copying
 * the image to the tensor's device address equals qmm_tensor_set of all of
 * its bytes. */
int    qmm_tensor_pack(int32_t type, const int64_t ne[4], const void * gguf, void * image, size_t image_size);
int    qmm_tensor_unpack(int32_t type, const int64_t ne[4], const void * image, void * gguf, size_t gguf_size);

/* ---- ops --------------------------------------------------------------- */
/* 1 when the op is taken; otherwise 0 and, if reason != NULL, why. */
int    qmm_supports_op(qmm_ctx * ctx, int32_t op, const qmm_tensor * src0, const qmm_tensor * src1,
                       const qmm_tensor * ids, const qmm_tensor * dst, char * reason, size_t reason_len);

/* Enqueue on the context's stream; asynchronous (call qmm_synchronize). */
int    qmm_mul_mat(qmm_ctx * ctx, const qmm_tensor * src0, const qmm_tensor * src1, const qmm_tensor * dst);
int    qmm_mul_mat_id(qmm_ctx * ctx, const qmm_tensor * src0, const qmm_tensor * src1,
                      const qmm_tensor * ids, const qmm_tensor * dst);
/* The FFN's gate/up pair and its GLU in one call: dst = act(gate x src1) * (up x src1), act =
 * enum qmm_glu, gate and up quantized [K, M, ne02, ne03] of one shape, src1 / dst as MUL_MAT's.
 * Replaces MUL_MAT, MUL_MAT, GLU (split form), the node chain the reference's fuse_mm_glu
 * matches (P01:65; ggml-opencl.cpp:9836-9878 by the reference's audit,
 * docs/campaigns/research-concept-mining/ipex-llm/audit.md:83-87).  One activation
 * quantization serves both; at GEMV widths with one batch and one weight type both matrices
 * stream in one launch.  Within MUL_MAT's tolerance of the unfused chain. */
int    qmm_mul_mat_glu(qmm_ctx * ctx, const qmm_tensor * gate, const qmm_tensor * up, const qmm_tensor * src1,
                       const qmm_tensor * dst, int32_t glu_op);
/* The MoE form: dst = act(MUL_MAT_ID(gate, src1, ids)) * MUL_MAT_ID(up, src1, ids), gate and
 * up expert stacks [K, M, n_as] of one type and shape, src1 / ids / dst as qmm_mul_mat_id's.
 * Replaces MUL_MAT_ID, MUL_MAT_ID, GLU (the reference's MUL_MAT_ID / GLU fuse, by its audit
 * docs/campaigns/research-concept-mining/ipex-llm/audit.md:83-87): one quantization, one
 * route, one GEMV launch over both stacks; experts averaging the grouped GEMM's pair count
 * (QMM_MOE_GEMM_MIN) take it twice, the GLU applied at the up product's stores.  Invalid ids
 * give zero rows. */
int    qmm_mul_mat_id_glu(qmm_ctx * ctx, const qmm_tensor * gate, const qmm_tensor * up, const qmm_tensor * src1,
                          const qmm_tensor * ids, const qmm_tensor * dst, int32_t glu_op);
/* qmm_mul_mat with nothing allocated: no reference counterpart; for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same operands as qmm_mul_mat and the same results within MUL_MAT's
 * tolerance, on the same kernels except that it never takes the K-split one-launch GEMV
 * ("gemv-fq" with work-groups meeting in the exchange tree, whose slots the context allocates):
 * such products run the activation pre-pass and the GEMV instead; the activation
 * quantization goes to a device array of QMM_NOALLOC_SCRATCH_BYTES that the library holds on
 * every GPU it runs on until the process ends (its address is looked up when a context is
 * created) instead of the context's scratch, and no graph dedup or kernel timing applies.
 * Fails with QMM_ERR_NOMEM, before launching anything, when src1's quantized activations need
 * more than that: about K * N * 1.2 bytes (K rounded up to 256; 16 MiB holds 512 columns at
 * K = 17408).  Every call on one GPU shares the array, which keeps the last call's contents:
 * calls that overlap on one GPU (contexts with different streams) race; calls on one context
 * are ordered by its stream. */
#define QMM_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int    qmm_mul_mat_noalloc(qmm_ctx * ctx, const qmm_tensor * src0, const qmm_tensor * src1, const qmm_tensor * dst);
/* Runs the nodes in order; bumps the graph generation first, so one
 * activation quantization serves every node of the graph that reads the same
 * src1 with the same vec_dot type. */
int    qmm_graph_compute(qmm_ctx * ctx, const qmm_node * nodes, int n_nodes);

/* HIP-graph capture and replay: no reference counterpart (the reference's OpenCL backend
 * launches every op on its queue); for callers whose decode steps are bound by launch latency,
 * the role CUDA graphs play in ggml-cuda's decode path.  qmm_capture_begin starts capturing
 * the context's stream; every op up to qmm_capture_end is recorded, not run.  While capturing
 * an op allocates nothing: it fails with QMM_ERR_NOMEM when the context's scratch is too small
 * for it (run the same ops once outside a capture first), records no kernel-timing events, and
 * counts its downgrades once.  The ops that synchronize (tensor set/get, qmm_synchronize,
 * qmm_quantize_act, buffer free) must not be called while capturing.  qmm_capture_end ends the
 * capture and, if every captured op succeeded, returns the instantiated graph; the stream is
 * usable again either way.  qmm_graph_launch replays it on the context's stream: the same
 * kernels on the same buffers (the data in them may change between launches).  The graph uses
 * the context's scratch: replays are ordered with the context's other work by its stream, and
 * an op run outside the graph may leave the scratch holding other activations, which the next
 * replay overwrites before it reads them.  An op outside the graph that needs more scratch than
 * the context has replaces the scratch: the graphs captured before then are refused by
 * qmm_graph_launch (QMM_ERR_INVALID; capture again), as is a graph launched on a context other
 * than its own.  Free the graph before its context. */
typedef struct qmm_graph qmm_graph;
int    qmm_capture_begin(qmm_ctx * ctx);
int    qmm_capture_end(qmm_ctx * ctx, qmm_graph ** out);
int    qmm_graph_launch(qmm_ctx * ctx, const qmm_graph * graph);
void   qmm_graph_free(qmm_graph * graph);

/* dst (f32, contiguous, ne = src ne) = dequantize_row_<type>(src) */
int    qmm_dequantize(qmm_ctx * ctx, const qmm_tensor * src, const qmm_tensor * dst);
/* Quantize f32 src [K, N] (rows of K) with ggml-cpu's from_float for
 * act_type (QMM_TYPE_Q8_0 or QMM_TYPE_Q8_K) and write the ggml block bytes
 * (block_q8_0 / block_q8_K, N*K/bs blocks) to host memory `out`. */
int    qmm_quantize_act(qmm_ctx * ctx, int32_t act_type, const qmm_tensor * src, void * out, size_t out_size);

int    qmm_synchronize(qmm_ctx * ctx);

/* ---- MoE router and combine -------------------------------------------- */
/* The router of a softmax-gated MoE layer in one kernel, replacing
 * llama.cpp's SOFT_MAX, ARGSORT (desc), VIEW, GET_ROWS, SUM_ROWS, CLAMP, DIV,
 * RESHAPE chain (the reference's fused kernel_topk_moe_softmax_norm,
 * P09:899-1000, matched at P02:786-821): for every token t (column of
 * logits [n_expert, T], f32), the softmax over its logits, the k largest
 * probabilities in descending order (ties: the lower expert) into
 * ids [k, T] (i32, the ids MUL_MAT_ID takes) and those probabilities divided
 * by their sum clamped to [cmin, cmax] into weights [k, T] (f32).
 * n_expert <= 1024, 1 <= k <= min(32, n_expert). */
int    qmm_moe_topk(qmm_ctx * ctx, const qmm_tensor * logits, const qmm_tensor * ids, const qmm_tensor * weights,
                    float cmin, float cmax);
/* The experts' outputs combined (llama.cpp's build_moe_ffn: MUL by the
 * weights, then the ADDs over the k slots, then the shared expert times the
 * sigmoid of its gate): dst[:, t] = sum_j weights[j, t] experts[:, j, t]
 * (+ shared[:, t] * sigmoid(gate[0, t])), each product rounded and the sums
 * taken slot by slot in order.  experts [M, k, T] (the MUL_MAT_ID dst),
 * weights [k, T], shared and dst [M, T], gate [1, T]; shared and gate both
 * or neither (NULL). */
int    qmm_moe_combine(qmm_ctx * ctx, const qmm_tensor * experts, const qmm_tensor * weights,
                       const qmm_tensor * shared, const qmm_tensor * gate, const qmm_tensor * dst);
/* A MoE FFN block in two launches (below 16 tokens; from 16, five after the router's):
 * llama.cpp's build_moe_ffn from the router's logits (or its ids and weights) on: the router
 * (SOFT_MAX, ARGSORT, GET_ROWS, SUM_ROWS, CLAMP, DIV, as qmm_moe_topk), MUL_MAT_ID gate and
 * up, the GLU, MUL_MAT_ID down, MUL by the weights, the ADDs over the slots, with an optional
 * shared expert (its gate and up MUL_MATs, GLU, down MUL_MAT,
 * times the sigmoid of its gate logit, added last) - the chain the reference runs node by node
 * (its fused router kernel_topk_moe_softmax_norm P09:899-1000, the gate/up/down MUL_MAT_IDs at
 * P01:1189-1248 with the GLU of fuse_mm_glu, the weights' MUL and ADDs on its element-wise
 * kernels) and that qmm_moe_topk, qmm_mul_mat_id_glu, qmm_mul_mat_id, qmm_mul_mat_glu,
 * qmm_mul_mat and qmm_moe_combine run as six dependent launches:
 *   dst[:, t] = sum_j weights[j, t] down[ids[j, t]] glu(gate[ids[j, t]] x_t, up[ids[j, t]] x_t)
 *               (+ sigmoid(shared_logit[0, t]) shared_down glu(shared_gate x_t, shared_up x_t))
 * with each weight product rounded and the slots added in slot order, the shared row last (the
 * graph's ADD order), or, when the down launch has fewer than 256 (tile, token) work-groups, in a
 * pairwise tree (equal to qmm_moe_combine's to float rounding).  With logits (f32 [n_as, T]) the ids and
 * weights are outputs, written with qmm_moe_topk's values (cmin / cmax clamp the winners' weight
 * sum; n_as <= 1024, n_used <= 32); without, they are inputs.  gate and up experts [K, M, n_as],
 * down [M, n_out, n_as], one type; x f32 [K, T] or [K, 1, T]; ids i32 and weights f32
 * [n_used, T]; the shared expert all three of shared_gate / shared_up [K, M] and shared_down
 * [M, n_out] of the experts' type, or none; shared_logit f32 [1, T] or NULL (the shared expert
 * unweighted); dst f32 [n_out, T] or [n_out, 1, T].  A negative id adds nothing, an id >= n_as
 * adds nothing and raises QMM_ERR_INVALID at the next qmm_synchronize.  From 16 tokens
 * (QMM_MOE_DIRECT_T) the block runs as routes: the router, then gate/up + GLU and down as expert
 * tasks with the shared expert one more slot of every token, then the combine in slot order
 * (qmm_moe_combine's sums).  Returns QMM_ERR_UNSUPPORTED (nothing enqueued) when the shared
 * expert's type or shapes differ from the experts', or when the experts average the pair count
 * from which MUL_MAT_ID takes the grouped GEMM (QMM_MOE_GEMM_MIN): then run the ops one by one.
 * The reference has no one call for the block: a ggml backend adaptor matches the node chain
 * (from the router's SOFT_MAX to the last ADD) and makes this call in its place. */
typedef struct qmm_moe_ffn_args {
    const qmm_tensor * gate_exps;      /* [K, M, n_as] */
    const qmm_tensor * up_exps;        /* [K, M, n_as] */
    const qmm_tensor * down_exps;      /* [M, n_out, n_as] */
    const qmm_tensor * x;              /* f32 [K, T] or [K, 1, T] */
    const qmm_tensor * logits;         /* NULL, or f32 [n_as, T]: then ids and weights are written */
    float              cmin, cmax;     /* the router's clamp of the winners' weight sum (with logits) */
    const qmm_tensor * ids;            /* i32 [n_used, T] */
    const qmm_tensor * weights;        /* f32 [n_used, T] */
    const qmm_tensor * shared_gate;    /* [K, M] or NULL */
    const qmm_tensor * shared_up;      /* [K, M] or NULL */
    const qmm_tensor * shared_down;    /* [M, n_out] or NULL */
    const qmm_tensor * shared_logit;   /* f32 [1, T] or NULL */
    int32_t            glu_op;         /* QMM_GLU_* */
    const qmm_tensor * dst;            /* f32 [n_out, T] or [n_out, 1, T] */
} qmm_moe_ffn_args;
int    qmm_moe_ffn(qmm_ctx * ctx, const qmm_moe_ffn_args * args);

/* ---- observability and timing ----------------------------------------- */
/* Ops that took a slower path than their weight type promises (the reference's DOWNGRADE keys,
 * ggml_backend_opencl_downgrades, 0100-...patch:19-22 and :67-80): `buf` (NUL-terminated,
 * truncated to buf_len) gets one "src=qmm <key>\t<count>\n" line per key, the key naming the
 * op, weight type, K, a column bucket, the path taken and the reason ("op=MUL_MAT type=Q5_K
 * k=5120 cols=2-8 path=gemv reason=no-mfma-gemv"); returns the total count over all keys. */
int64_t qmm_downgrades(qmm_ctx * ctx, char * buf, size_t buf_len);
/* Name of the kernel path the last op took.  MUL_MAT: "gemv" (activation pre-pass + v_dot4
 * GEMV, 1..8 columns per weight pass), "gemv-mfma" (pre-pass + the few-column int8 MFMA GEMV,
 * up to 32 columns per weight pass), "gemv-fq" (one launch: the GEMV quantizes its own
 * activations, K split over work-groups met in an exchange tree), "gemm-stream" (tiled pre-pass
 * + the streaming int8 MFMA GEMM), "gemm-mfma" (pre-pass + the shared-tile int8 MFMA GEMM).
 * MUL_MAT_ID: "gemv-id-fq" (one launch, each (slot, token) pair read from ids), "gemv-id" /
 * "gemv-id-mfma" (route + expert tasks on either GEMV), "gemm-id-stream" (route + the grouped
 * streaming GEMM).  qmm_mul_mat_glu: "glu-fused-gemv-fq", "glu-fused-gemv", "glu-fused-gemv-mfma"
 * (gate and up in one launch) or "glu-" + the MUL_MAT path (two products and a GLU kernel).
 * qmm_mul_mat_id_glu: "glu-gemv-id-fq", "glu-gemv-id", "glu-gemv-id-mfma", "glu-gemm-id-stream"
 * (route + the grouped GEMM for gate, then for up with the GLU at its stores).  The router and
 * the combine: "moe-topk", "moe-combine"; qmm_moe_ffn: "moe-ffn-fq" (below 16 tokens),
 * "moe-ffn-route". */
const char * qmm_last_path(qmm_ctx * ctx);

/* The launch a qmm_mul_mat with these tensors would make (host only, no
 * device, no buffers needed: only types and shapes are read). */
typedef struct qmm_launch_info {
    char    path[32];          /* as qmm_last_path: "gemv", "gemv-mfma", "gemv-fq", "gemm-stream" or
                                  "gemm-mfma" */
    int64_t workgroups;
    int32_t threads;           /* per work-group */
    int32_t cols_per_task;     /* GEMV: activation columns per weight pass */
    int64_t tasks;
    int32_t k_waves;           /* GEMV: waves per work-group, splitting K */
    int32_t k_slices;          /* GEMV: work-groups per 64-row tile, splitting K */
    int32_t groups_per_wave;   /* GEMV: 256-weight groups per wave */
    int64_t lds_bytes;         /* dynamic LDS per work-group */
    int32_t tiles_per_wg;      /* GEMV: 64-row tiles per work-group ("gemv-mfma": threads / 64 =
                                  tiles_per_wg x k_waves) */
} qmm_launch_info;
int    qmm_describe_mul_mat(const qmm_tensor * src0, const qmm_tensor * src1, const qmm_tensor * dst,
                            qmm_launch_info * out);

/* HIP events on the context's stream: begin records, end records and waits,
 * returning the elapsed milliseconds (device time between the two). */
int    qmm_timer_begin(qmm_ctx * ctx);
float  qmm_timer_end(qmm_ctx * ctx);

/* Per-kernel device time of the main kernel of every op (the GEMV / GEMM,
 * not the activation pre-pass): enable = 1 clears and starts stamping a HIP
 * event pair with each such kernel's own start and end (the dispatch itself,
 * as a profiler reports it); enable = 2 instead records the pair on the
 * stream right before and right after the launch (the start completes with
 * the work queued ahead of the kernel); 0 stops.  qmm_kernel_time waits for
 * the stream and returns the summed milliseconds and the launch count;
 * qmm_kernel_times writes each launch's milliseconds (at most cap) and
 * returns the launch count, -1 on error. */
int    qmm_kernel_timing(qmm_ctx * ctx, int enable);
int    qmm_kernel_time(qmm_ctx * ctx, double * total_ms, int64_t * launches);
int64_t qmm_kernel_times(qmm_ctx * ctx, double * ms, int64_t cap);

/* Copy between device buffers on the context's stream (harness plumbing). */
int    qmm_buffer_copy(qmm_ctx * ctx, qmm_buffer * dst, size_t dst_off, const qmm_buffer * src, size_t src_off, size_t size);

#ifdef __cplusplus
}
#endif

#endif /* QMM_H */
