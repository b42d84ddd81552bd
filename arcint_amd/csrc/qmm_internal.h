// qmm_internal.h - layouts and launch interfaces shared by the libqmm host
// code and its HIP kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/qmm.h"

// QMM_RED = k plants known mistake k in one kernel family (a mutation build of the tests,
// arcint_amd.build --red k, never the product: the product build leaves it 0); the GPU parity
// suite must fail against every k (tests/red/run_red.py).  1 dequant, 2 q8_0 quantizer,
// 3 v_dot4 GEMV, 4 MFMA GEMV, 5 Q4_K GEMM, 6 streaming GEMM, 7 MoE route, 8 fused MoE GEMV.
#ifndef QMM_RED
#define QMM_RED 0
#endif

namespace qmm {

// ---------------------------------------------------------------------------
// Weight image in HBM (the device layout behind qmm_tensor_set/get).
//
// Rows of every matrix (expert / 2-D slice) are grouped in tiles of 64 rows
// and the K axis in groups of 256 weights (8 GGUF blocks of Q4_0/Q8_0, one
// super-block of the K-quants; a last partial group of Q4_0/Q8_0 is padded
// with zero blocks).  The bytes of one (tile, group) - a "tile-group" - are
// contiguous and consist of `nchunk` chunk planes of 64 x 16 bytes (row r of
// the tile at byte 16 r of every plane) followed by an optional tail plane of
// 64 x `tail` bytes.  A wave that gives lane r the row r reads one chunk
// plane with a single fully coalesced 1 KB load.  Planes per tile-group:
//   Q4_0    chunk p < 8: qs of block p | chunk 8: d of blocks 0..7 (fp16)
//   Q8_0    chunks 2p, 2p+1: qs[0:16], qs[16:32] of block p | chunk 16: d[8]
//   Q4_K    chunk c < 8: qs[16c:16c+16] | chunk 8: {d, dmin, scales[12]}
//   Q5_K    as Q4_K | chunks 9, 10: qh[0:16], qh[16:32]
//   Q6_K    chunk c < 8: ql[16c:+16] | chunks 8..11: qh[16c:+16] |
//           chunk 12: scales[16] | tail (2 B): d
//   IQ4_XS  chunk c < 8: qs[16c:+16] | tail (8 B): {d, scales_h, scales_l[4]}
//   IQ4_NL  as Q4_0 (the same block bytes; the codes index the codebook)
// Tile-groups are stored [matrix][tile][group]; rows past M in the last tile
// and the padding blocks of a partial group are zero bytes.
// ---------------------------------------------------------------------------
constexpr int kTileRows = 64;
constexpr int kGroupW = 256;
constexpr int kChunk = 1024;
constexpr size_t kPlaneAlign = 256;
static inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// bytes of one tile-group: chunk planes * 1 KB + 64 rows * tail bytes (0: not a weight type)
__host__ __device__ constexpr int tile_group_bytes(int type) {
    return type == QMM_TYPE_Q4_0 || type == QMM_TYPE_IQ4_NL ? 9 * kChunk
         : type == QMM_TYPE_Q8_0                          ? 17 * kChunk
         : type == QMM_TYPE_Q4_K                          ? 9 * kChunk
         : type == QMM_TYPE_Q5_K                          ? 11 * kChunk
         : type == QMM_TYPE_Q6_K                          ? 13 * kChunk + 2 * kTileRows
         : type == QMM_TYPE_IQ4_XS                        ? 8 * kChunk + 8 * kTileRows
                                                          : 0;
}

// The GEMV kernels keep their weight loads unconditional: a stage past the end of a wave's
// range reads this many bytes of zeros (the context's sink) instead of weights.  A stage reads
// at most one tile-group from its base, so every type's tile-group must fit in the sink.
constexpr size_t kSinkBytes = 32768;
static_assert(tile_group_bytes(QMM_TYPE_Q4_0) <= (int)kSinkBytes && tile_group_bytes(QMM_TYPE_Q8_0) <= (int)kSinkBytes &&
                  tile_group_bytes(QMM_TYPE_Q4_K) <= (int)kSinkBytes && tile_group_bytes(QMM_TYPE_Q5_K) <= (int)kSinkBytes &&
                  tile_group_bytes(QMM_TYPE_Q6_K) <= (int)kSinkBytes && tile_group_bytes(QMM_TYPE_IQ4_XS) <= (int)kSinkBytes &&
                  tile_group_bytes(QMM_TYPE_IQ4_NL) <= (int)kSinkBytes,
              "a stage load past the end reads one tile-group's extent of the sink");

struct TypeLayout {
    int type;
    int blck;     // weights per GGUF block
    int bytes;    // GGUF bytes per block
    int bpg;      // GGUF blocks per 256-weight group
    int nchunk;   // chunk planes per tile-group
    int tail;     // bytes per row of the tail plane (0: none)
    int tg;       // bytes per tile-group = nchunk * 1024 + 64 * tail
};

const TypeLayout * type_layout(int type);   // nullptr for unknown types

struct ImageShape {
    int64_t K, M, nmat;   // row length, rows per matrix, matrices (ne2 * ne3)
    int64_t bpr;          // GGUF blocks per row
    int64_t G;            // 256-weight groups per row
    int64_t ntiles;       // 64-row tiles per matrix
    size_t bytes;         // image bytes (a multiple of 256)
};
// false when ne[0] is not a whole number of blocks
bool image_shape(const TypeLayout & L, const int64_t ne[4], ImageShape * s);

// One piece of a GGUF block placed in a tile-group: `size` bytes from byte
// `src` of the block go to byte `dst` of the tile-group (row 0, block slot 0);
// row r adds r * row_step, block slot p (Q4_0/Q8_0) adds p * slot_step.
struct Piece { int src, size, dst, row_step, slot_step; };
int block_pieces(const TypeLayout & L, Piece out[16]);

// ---------------------------------------------------------------------------
// Quantized activations (the vec_dot type's from_float, done on the device).
// Columns are padded to ldk = K rounded up to 256 (zero codes, zero scales,
// zero sums past K).  For column c of ncols:
//   codes  int8 [c][ldk]
//   d      f32  [c][ldk/bs]     bs = 32 (q8_0) or 256 (q8_K); q8_0's d is
//                               the fp16-rounded scale widened to f32
//   sums   i16  [c][ldk/ss]     ss = 32 (q8_0: sum of the block's codes)
//                               or 16 (q8_K: ggml's bsums)
// ---------------------------------------------------------------------------
struct ActBuf {
    int8_t *   codes;
    float *    d;
    int16_t *  sums;
    float *    dT;         // non-null: the scales again, block-major: dT[b * ldT + c]
    int8_t *   bsp;        // q8_K: per super-block sb and column c, 16 bytes at (sb * ldT + c) * 16:
                           // the 8 sub-block sums (32 codes each) split as 64 bh + bl, bh[8] then bl[8]
    int64_t    ldT;        // >= ncols + 64 (the GEMM reads whole 64-column tiles); set also without dT
    int64_t    K;
    int64_t    ldk;        // K rounded up to 256
    int64_t    ncols;
    int        vdt;        // QMM_TYPE_Q8_0 or QMM_TYPE_Q8_K
};

// Zeroing of dst columns by the activation pre-pass (the GEMV then adds the
// partial sums of its K slices with atomics): column c = (i1, i2, i3), i1
// fastest, floats [0, M) at i1 * nb1 + i2 * nb2 + i3 * nb3 (float strides).
struct ZeroJob {
    float * dst;
    int64_t M, ncols, ne1, ne2;     // rows [m0, M) of each column
    int64_t nb1, nb2, nb3;
    int64_t m0;                     // 0 unless set
};

__host__ __device__ static inline int act_block(int vdt) { return vdt == QMM_TYPE_Q8_0 ? 32 : 256; }
__host__ __device__ static inline int act_sum_block(int vdt) { return vdt == QMM_TYPE_Q8_0 ? 32 : 16; }
__host__ __device__ static inline int vec_dot_type(int type) {
    return (type == QMM_TYPE_Q4_0 || type == QMM_TYPE_Q8_0 || type == QMM_TYPE_IQ4_NL) ? QMM_TYPE_Q8_0 : QMM_TYPE_Q8_K;
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
    const uint8_t * base;      // image of matrix 0
    int64_t M;                 // rows per matrix
    int64_t K;                 // weights per row
    int64_t bpr;               // GGUF blocks per row
    int64_t G;                 // groups per row
    int64_t ntiles;            // tiles per matrix
    int tg;                    // bytes per tile-group
};

// tile-group (mat, tile, g) of the image
__host__ __device__ static inline const uint8_t * tile_group(const WView & w, int64_t mat, int64_t tile, int64_t g) {
    return w.base + (size_t)(((mat * w.ntiles + tile) * w.G + g)) * (size_t)w.tg;
}

// A routed task: up to TC columns against one weight matrix.  GEMV tasks carry up to 8; the
// grouped MoE GEMM's units 64 (one 64-column wave job of the streaming Q4_K GEMM).
// A column's activation id and dst offset lie together, so the route writes each pair with one
// 16-byte store (it scatters every pair of a MUL_MAT_ID from one work-group, and its time goes to
// those stores).
struct TaskCol {
    int32_t col;                   // activation column id
    int32_t pad;
    int64_t dst_off;               // float offset of dst row 0 for that column
};
template <int TC> struct TaskOf {
    int32_t mat;                   // weight matrix (expert / slice) index; <0: zero rows
    int32_t ncols;
    TaskCol c[TC];
};
constexpr int kMaxTaskCols = 8;
constexpr int kUnitCols = 64;
using GemvTask = TaskOf<kMaxTaskCols>;
using GemmUnit = TaskOf<kUnitCols>;

// ---------------------------------------------------------------------------
// Launchers (defined in the .hip files); all enqueue on `s`.  A non-null
// KTime has its events stamped with the main kernel's own start and end (the
// dispatch itself, as a profiler sees it).
// ---------------------------------------------------------------------------
struct KTime {
    hipEvent_t start, stop;
};
hipError_t launch_dequant(int type, const WView & w, int64_t nmat, float * y, hipStream_t s);
hipError_t launch_quantize(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, const ZeroJob * z,
                           hipStream_t s);
// writes ggml block bytes (block_q8_0 / block_q8_K) of an ActBuf into `out` (device)
hipError_t launch_act_to_blocks(const ActBuf & a, void * out, hipStream_t s);

// Dense MUL_MAT batch description (columns of one batch are contiguous ids)
struct GemvDense {
    int64_t ne11, ne12, ne13, r2, r3, ne02;
    int64_t d_nb1, d_nb2, d_nb3;   // dst strides in floats
    // gate/up in one launch: matrix 1 is the image at base2 (same shape and type as matrix 0),
    // and batch b reads activation columns b * col_bs + i1 (0: every batch the same columns)
    const uint8_t * base2 = nullptr;
    int64_t col_bs = -1;           // -1: ne11
};

// Launch shape of a GEMV (host): W waves per work-group and KS work-groups
// per 64-row tile split K, spw groups of 256 weights per wave.  KS > 1 adds
// partial sums to dst with atomics, so dst must be zeroed first.
// v_dot4 kernel: a work-group is W waves splitting K on one tile (spw groups each), KS
// work-groups per tile.  MFMA kernel (mma): a work-group is tw tiles x W / tw waves splitting
// K; it stages its K range's activations in LDS (kMmaColBytes per column and group, at most
// kMmaMaxGroups groups).
struct GemvPlan {
    int nc;                        // columns per task (1..8; mma: 1..kMmaMaxCols)
    int64_t ntasks;                // grid tasks (list mode: upper bound)
    int W, KS, spw;
    bool mma;                      // dots on the MFMA (few columns; Q4_0, Q8_0, Q4_K, IQ4_XS, IQ4_NL)
    int tw;                        // mma: tiles per work-group, W / tw waves of each split K
    int cm;                        // mma: the kernel's columns per task (8, 16 or 32) >= nc
};
constexpr int kMmaColBytes = 272;  // 256 codes + 16 bytes of padding (LDS banks)
constexpr int kMmaZeroBytes = 256; // zeros ahead of the codes
constexpr int kMmaMaxGroups = 24;  // groups a work-group stages at 8 columns (8 / cm of it at cm)
constexpr int kMmaMaxCols = 32;    // columns of one MFMA task (the A operand's 32 rows)
// want_mma: use the MFMA kernel where the type allows it
bool gemv_plan(int type, const WView & w, int nc, int64_t ntasks, bool allow_split, bool want_mma, GemvPlan * plan);
int64_t gemv_workgroups(const WView & w, const GemvPlan & plan);
// The weight loads of a GEMV launch, replayed on the host (no device) with the kernels' own
// index functions: byte ranges relative to the image base of `nmat` matrices, and of the sink.
// Task lists take matrix list_mat for every task (dense launches derive it from `dense`).
struct GemvExtent {
    int64_t image_bytes;        // bytes of the nmat matrices' tile-groups
    int64_t real_lo, real_hi;   // lowest first byte / highest end of a load from the image
    int64_t sink_hi;            // highest end of a load from the sink (<= kSinkBytes)
    int64_t real_loads, sink_loads;
    int64_t read_end;           // bytes a stage reads from its tile-group base
    int64_t bad;                // loads outside the image or the sink, groups outside [0, G)
};
bool gemv_extent(int type, const WView & w, const GemvPlan & plan, const GemvDense * dense, int64_t nmat, int list_mat,
                 GemvExtent * e);
size_t gemv_lds_bytes(int type, const GemvPlan & plan);
// whether the few-column MFMA kernel handles this weight type
bool gemv_mma_supported(int type);

// GEMV: dst[dst_off + m] for m < M, rows of matrix `mat` of each task, from
// the pre-pass activations `a` (ldk == 256 * groups).  List mode (tasks !=
// nullptr): `ntasks_dev` (optional) bounds the task list on the device.
// Dense mode (tasks == nullptr): tasks of up to nc columns from `dense`.
// `sink`: kSinkBytes of device memory the kernel may read (not write) for
// loads past the end of its pipeline.
// pair (task lists only), a second expert stack of w's shape at pair->base2: with glu < 0 the
// list runs a second time on it, its dst offsets plus up_doff floats (plan.ntasks counts both
// passes); with glu >= 0 (enum qmm_glu) each work-group streams its tile of both stacks and
// stores act(gate) * up
struct GemvPair {
    const uint8_t * base2;
    int64_t up_doff;
    int glu = -1;
    // list mode: tasks of matrix sh_mat read the shared expert's images instead (sh_base, and
    // sh_base2 for base2's); -1: none
    int32_t sh_mat = -1;
    const uint8_t * sh_base = nullptr;
    const uint8_t * sh_base2 = nullptr;
};
hipError_t launch_gemv(int type, const WView & w, const GemvPlan & plan, const ActBuf & a, const GemvTask * tasks,
                       const int32_t * ntasks_dev, const GemvDense * dense, float * dst, const void * sink,
                       hipStream_t s, const KTime * kt = nullptr, const GemvPair * pair = nullptr);

// The v_dot4 GEMV with its own activation quantization (k_gemv_fq): no pre-pass, K split
// among the W waves of a work-group (at most 16) and, for dense products, over KS
// work-groups per tile whose sums meet in a tree of exchanges (tree slots below); every
// output is stored once.  nc = columns per task (1 or 2).  Dense tasks as GemvDense; with ids,
// task p is the MUL_MAT_ID pair p = t n_used + i (nc = 1).  glu >= 0: the work-group streams w
// (gate) then base2 (up) and stores act(gate) * up.
struct FusedGemv {
    F32Cols x;                  // src1's f32 columns
    int64_t K;
    GemvDense dense;            // dense tasks (ids == nullptr)
    const char * ids;           // MUL_MAT_ID: i32 ids, pair (i, t) at t ids_nb1 + i ids_nb0 bytes
    int64_t ids_nb0, ids_nb1, n_used, T, ne11, n_as;
    int64_t dnb1, dnb2;         // dst floats of pair (i, t): t dnb2 + i dnb1
    int32_t * bad_id;           // set when an id is >= n_as
    const uint8_t * base2;      // glu >= 0: the up image
    int glu;
    uint32_t * tree;            // KS > 1: gemv_fused_tree_words words, each kTreeEmpty; combine:
                                // T x ntiles x 2 (n_used + n_shared) x 64 words
    // MoE FFN (ids != nullptr): a shared-expert slot n_used of every token (n_shared = 1) with
    // images sh_base (gate / only matrix) and sh_base2 (up) of w's shape; comb: pair (i, t)'s row
    // times cw[t cw_nb1 + i cw_nb0] (the shared slot: sigmoid(sl[t sl_nb1]), 1 without sl), the
    // token's slots added and stored at dst + t d_nb1: comb 1 in the tree (grid: tiles x slots x
    // tokens), comb 2 in slot order through LDS (grid: tiles x 1 x tokens, one wave per slot over
    // the whole K: plan W = slots, spw >= G)
    int n_shared;
    const uint8_t * sh_base;
    const uint8_t * sh_base2;
    int comb;
    const float * cw;
    int64_t cw_nb0, cw_nb1;
    const float * sl;
    int64_t sl_nb1, d_nb1;
    // gate/up with the router (lg != nullptr): every work-group's first wave ranks token t's
    // logits lg + t lg_nb1 (n_expert of them, top n_used, weight sum clamped to [cmin, cmax]);
    // the ids go to `ids` (written, ids_nb0 == 4) and the weights to wout + t wout_nb1
    const float * lg;
    int64_t lg_nb1;
    int n_expert;
    float cmin, cmax;
    float * wout;
    int64_t wout_nb1;
};
struct FusedPlan {
    int nc, W, spw;
    int KS = 1;                 // work-groups per tile along K (dense)
    int64_t ntasks;
    int64_t lds;
};
// The slots of the K-slice tree hold this between launches: a signaling NaN, which no float
// arithmetic produces, so a slot holds either it or one work-group's sum.  A launch leaves
// every slot it touched at this value again.
constexpr uint32_t kTreeEmpty = 0x7F800001u;
// about `target` waves over ntasks x tiles work-groups; false when the K range does not fit
bool gemv_fused_plan(int type, const WView & w, int nc, int64_t ntasks, int target, FusedPlan * plan);
// dense products split along K: work-groups of W waves with spw groups per wave, KS =
// ceil(G / (W spw)) >= 2 of them per tile; false when that gives one slice or does not fit
bool gemv_fused_split_plan(int type, const WView & w, int nc, int64_t ntasks, int W, int spw, FusedPlan * plan);
// MoE down with the combine in slot order (comb 2): a work-group per (tile, token) of nslots waves,
// each over the whole K; false when the slots exceed a work-group's waves or the LDS
bool gemv_fused_slot_plan(int type, const WView & w, int64_t nslots, int64_t T, FusedPlan * plan);
// tree slots (32-bit words) a split plan needs (glu: gate and up sums travel as one 64-bit pair)
int64_t gemv_fused_tree_words(const WView & w, const FusedPlan & plan, bool glu);
int gemv_fused_waves_target();
hipError_t launch_gemv_fused(int type, const WView & w, const FusedPlan & plan, const FusedGemv & f, float * dst,
                             const void * sink, hipStream_t s, const KTime * kt = nullptr);

// Prefill GEMM (int8 MFMA, all five types): for every batch b < nbatch,
// dst[doff(b) + n * d_nb1 + m] = W(mat(b)) row m . activation column
// col0(b) + n, for n < N, m < M.  Activations come from the pre-pass with
// block-major scales (a.dT) and, for q8_K, the split sub-block sums (a.bsp).
struct GemmBatch {
    int64_t ne12, r2, r3, ne02;    // batch b = (i2, i3): mat = i2 / r2 + (i3 / r3) * ne02
    int64_t d_nb1, d_nb2, d_nb3;   // dst strides in floats
};
hipError_t launch_gemm(int type, const WView & w, const ActBuf & a, int64_t N, int64_t nbatch,
                       const GemmBatch & bt, float * dst, hipStream_t s, const KTime * kt = nullptr);
// ---------------------------------------------------------------------------
// Tiled activations of the streaming GEMM (k_gemm3), written by its pre-pass.
// The columns of each batch go in tiles of 32: column n of batch b is column
// n % 32 of tile b * ntb + n / 32 (ntb = ceil(N / 32)); columns past N in a
// batch's last tile hold zeros.  For tile t and 32-weight block k < nblk:
//   A  int8 [t][k][64][16]  the v_mfma_i32_32x32x32_i8 A operand: the 16
//      bytes of lane (i, h) are codes 16 h .. 16 h + 15 of the block in
//      column i (i = lane % 32, h = lane / 32)
//   D  f32 [t][k][32]       the q8_0 block scales (fp16-rounded, as ggml-cpu
//      keeps them) in the MFMA's output order: entry 16 h + r is column
//      8 (r / 4) + 4 h + r % 4, the column that register r of lane half h
//      holds
// ---------------------------------------------------------------------------
//   q8_K (the K-quant GEMM) keeps A as above (a 32-weight block is a sub-block) and per
//   256-weight super-block sb of tile t:
//   D  f32 [t][sb][32]      the super-block scale d in the same output order
//   S  int8 [t][sb][32][16] column i's 8 sub-block code sums split as 64 bh + bl: bh[8],
//      then bl[8] (the A operand of the Q4_K min term)
// ---------------------------------------------------------------------------
struct TiledAct {
    int8_t * A;
    float * D;
    int8_t * S;        // q8_K only
    int64_t nblk;      // 32-weight blocks per column (ldk / 32)
    int64_t ntb;       // tiles per batch
    int64_t ntiles;    // tiles of all batches
    int64_t N;         // columns per batch
    int vdt;           // QMM_TYPE_Q8_0 or QMM_TYPE_Q8_K
};
__host__ __device__ constexpr int tiled_pos(int i) { return 16 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3); }
// bytes of the two arrays for ntiles tiles of nblk blocks (each a multiple of 256)
__host__ __device__ inline size_t tiled_a_bytes(int64_t ntiles, int64_t nblk) { return (size_t)(ntiles * nblk) * 1024; }
__host__ __device__ inline size_t tiled_d_bytes(int64_t ntiles, int64_t nblk) { return (size_t)(ntiles * nblk) * 128; }
__host__ __device__ inline size_t tiled_s_bytes(int64_t ntiles, int64_t nblk) { return (size_t)(ntiles * nblk) * 64; }
// quantization of the f32 columns into the tiled layout (t.vdt: q8_0 or q8_K, ggml-cpu's
// from_float numerics)
hipError_t launch_quantize_tiled(const F32Cols & src, int64_t K, const TiledAct & t, hipStream_t s);

// Streaming GEMM for Q4_0, Q8_0, IQ4_NL (q8_0 activations) and Q4_K (q8_K): for
// every weight batch b < nbatch, dst[doff(b) + n d_nb1 + m] = W(mat(b)) row m .
// column n of batch b, n < N, m < M.  Each output is written once (no atomics,
// no zeroing of dst).
bool gemm3_supported(int type);
struct G3Shape {
    int C, U, KS, SB;              // column tiles per wave, row-unit waves per K slice, K slices, blocks per stage
    int R;                         // rows per wave (64: Q4_0 / Q8_0 / IQ4_NL, 32: Q4_K)
    int64_t mbn, nbn;              // work-group blocks along M and N per batch
    int sps, nst;                  // stages per K slice, stages along K
    int threads, lds;
    int64_t workgroups;            // all batches
    // the tail (the blocks past a whole number per CU): blocks [full, mbn nbn) run as ts
    // work-groups each, piece i over stages [i pk, (i + 1) pk) (the pieces meet in tree slots:
    // tslots per output and block); ts = 1: every block whole
    int64_t full;
    int ts, pk, tslots;
    int64_t fchunk, tchunk;        // per XCD: whole blocks, tail pieces
};
bool gemm3_shape(int type, const WView & w, int64_t N, int64_t nbatch, G3Shape * sh);
// tree words the tail pieces of that launch meet in (0: no pieces)
size_t gemm3_tree_words(const G3Shape & sh);
// Grouped MoE GEMM (MUL_MAT_ID with many pairs per expert): the route's 64-column units
// (*nunits of at most max_units) of one expert each, activations gathered from the route's q8_K
// quantization a; unit pairs with mat < 0 get zero rows.  Q4_K, Q6_K, Q5_K and IQ4_XS.
// dst_span: the floats from dst to one past its last element (below 2^30: the stores take
// 32-bit byte offsets).  With glu >= 0 (QMM_GLU_*) this is the up product of a gate/up pair:
// each stored value is act(gsrc[o]) * up at its dst offset o, gsrc the gate product's rows at
// the same offsets (zero rows stay zero).  one_slice: 4-wave one-slice blocks, three a CU
// (mostly full units, a block per CU or more), else the launch rule's shape.
bool gemm3_id_supported(int type);
bool gemm3_id_shape(const WView & w, int64_t max_units, bool one_slice, G3Shape * sh);
hipError_t launch_gemm3_id(int type, const WView & w, const ActBuf & a, const GemmUnit * units, const int32_t * nunits,
                           int64_t max_units, bool one_slice, float * dst, int64_t dst_span, hipStream_t s,
                           const KTime * kt = nullptr, const float * gsrc = nullptr, int glu = -1);
// tree: gemm3_tree_words(shape) words of tree slots, each kTreeEmpty (left so), or nullptr: then
// the tail blocks run whole
hipError_t launch_gemm3(int type, const WView & w, const TiledAct & a, int64_t nbatch, const GemmBatch & bt,
                        float * dst, hipStream_t s, const KTime * kt = nullptr, uint32_t * tree = nullptr);

// K slices the GEMM splits this product into; above 1 the slices add their
// partial sums to dst with atomics, so dst must be zeroed first.
int gemm_kslices(int type, const WView & w, int64_t N, int64_t nbatch);
// first dst row that K slices add into (the pre-pass zeroes rows [that, M) of every column;
// M: no row)
int64_t gemm_zero_from(int type, const WView & w, int64_t N, int64_t nbatch);
// launch shape of that GEMM (qmm_describe_mul_mat)
void gemm_shape(int type, const WView & w, int64_t N, int64_t nbatch, int64_t * workgroups, int * threads,
                int * lds_bytes);

// MoE routing: builds GEMV tasks (one per expert and up to 8 pairs) from ids.
struct RouteArgs {
    const int32_t * ids;        // [T][n_used] with row stride ids_nb1 (bytes)
    size_t ids_nb0, ids_nb1;
    int64_t n_used, T, ne11, n_as;
    int64_t dst_nb1, dst_nb2;   // float strides of dst dims 1 and 2
    int32_t * bad_id;           // set to 1 (a plain store) when an id is >= n_as
    int32_t shared = 0;         // 1: every token has one more slot, n_used, holding the shared
                                // expert (no id read): its pairs go to bucket n_as, tasks of
                                // matrix n_as; the invalid ids' bucket moves to n_as + 1
};
// MoE router: for each token t (logits column, n_expert <= 1024 floats at logits + t nbl1),
// ids [k] (i32 at ids + t nbi1) and weights [k] (f32 at w + t nbw1), k <= 32
struct TopkArgs {
    const char * logits;
    char * ids;
    char * w;
    int64_t nbl1, nbi1, nbw1;   // bytes
    int n_expert, k;
    int64_t n_tok;
    float cmin, cmax;
};
hipError_t launch_topk(const TopkArgs & a, hipStream_t s);
// MoE combine: dst[m, t] = sum_j w[j, t] experts[m, j, t] (+ shared[m, t] sigmoid(gate[t]));
// strides in bytes, elements along m contiguous
struct CombineArgs {
    const char * experts;
    const char * w;
    const char * shared;        // optional
    const char * gate;          // with shared: one logit per token
    char * dst;
    int64_t M, T;
    int k;
    int64_t enb1, enb2, wnb1, snb1, gnb1, dnb1;
};
hipError_t launch_combine(const CombineArgs & a, hipStream_t s);

// GLU of a gate/up pair: dst[m + n d_nb1 + i2 d_nb2 + i3 d_nb3] = act(gate[i]) * up[i], i over the
// contiguous [nb][N][M] of gate and up (batch b = i2 + i3 ne12)
struct GluArgs {
    const float * gate;
    const float * up;
    float * dst;
    int64_t M, N, nb, ne12;
    int64_t d_nb1, d_nb2, d_nb3;   // floats
};
hipError_t launch_glu(int op, const GluArgs & a, hipStream_t s);

// scratch: pairs [T*n_used]; tasks out
// tasks of mat = -1 carry pairs of invalid ids: the GEMV writes their dst rows as zeros
hipError_t launch_route(const RouteArgs & r, int32_t * scratch, GemvTask * tasks, int32_t * ntasks, hipStream_t s);
hipError_t launch_route(const RouteArgs & r, int32_t * scratch, GemmUnit * units, int32_t * nunits, hipStream_t s);
// the route and the activation quantization (no dst zeroing) in one launch
hipError_t launch_quant_route(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, const RouteArgs & r,
                              int32_t * scratch, GemvTask * tasks, int32_t * ntasks, hipStream_t s);
hipError_t launch_quant_route(const F32Cols & src, int64_t K, int64_t ncols, const ActBuf & a, const RouteArgs & r,
                              int32_t * scratch, GemmUnit * units, int32_t * nunits, hipStream_t s);

}  // namespace qmm

// Self-check for the tests, exported from libqmm but not part of the op ABI (include/qmm.h):
// the GEMV weight loads of a MUL_MAT / MUL_MAT_ID shape replayed on the host (qmm_api.cpp).
extern "C" int qmm_internal_gemv_extent(int32_t type, const int64_t ne0[4], int64_t N, int64_t nbatch,
                                        int64_t id_n_used, int64_t out[8]);
// The streaming GEMM's activation pre-pass for weights of `type` (q8_0 or q8_K tiles) over the
// f32 tensor src1, copied to host `out`: A, then D, then S (q8_K), as the kernel reads them.
// Returns the byte count written (0 on error; `cap` too small is an error).
extern "C" int64_t qmm_internal_quantize_tiled(struct qmm_ctx * ctx, const struct qmm_tensor * src1, int32_t type,
                                               void * out, int64_t cap);
