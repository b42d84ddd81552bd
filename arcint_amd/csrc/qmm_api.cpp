// qmm_api.cpp - the C ABI of libqmm (include/qmm.h): device context, buffers,
// GGUF <-> weight image repack, op validation and dispatch.  Host C++ calling HIP
// directly; one in-order stream per context, like one ggml backend.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "qmm_internal.h"
#include "qmm_layout.h"

using namespace qmm;

// The activation scratch of qmm_mul_mat_noalloc: a file-scope device array, one copy on every
// GPU the library runs on, held until the process ends.  Host code never uses the array's name
// as an address (on the host it is only a stand-in): it uses the per-device address that
// hipGetSymbolAddress returns at context creation (scratch_address below).
static __device__ __align__(256) uint8_t scratch[QMM_NOALLOC_SCRATCH_BYTES];

struct qmm_buffer {
    void * ptr = nullptr;
    size_t size = 0;
};

struct qmm_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    void * sink = nullptr;           // kSinkBytes of zeros the GEMV reads past the end of its pipeline
    int32_t * dflags = nullptr;      // device error flags: [0] an id >= n_as was routed
    int32_t * hflags = nullptr;      // pinned host copy, read by qmm_synchronize
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::string err;
    std::string path = "none";
    // activation scratch
    void * act = nullptr;
    size_t act_cap = 0;
    // activation dedup inside qmm_graph_compute
    uint64_t graph_gen = 0;
    bool in_graph = false;
    struct ActKey {
        const qmm_buffer * buf = nullptr;
        size_t offs = 0;
        int64_t ne[4] = { 0, 0, 0, 0 };
        size_t nb[4] = { 0, 0, 0, 0 };
        int vdt = 0;
        bool dT = false;
        bool tiled = false;          // the streaming GEMM's tiled layout (cached_tiled)
        uint64_t gen = 0;
        bool valid = false;
    } key;
    ActBuf cached{};
    TiledAct cached_tiled{};
    // MoE route scratch: ids copy, tasks, task count
    void * route = nullptr;
    size_t route_cap = 0;
    // the route in the scratch, reused inside one graph by products with the same ids, ne11,
    // dst strides and expert count (the reference's route cache, P01:1267-1269)
    struct RouteKey {
        qmm_tensor ids{};
        int64_t ne11 = 0, n_as = 0, dnb1 = 0, dnb2 = 0;
        int shared = 0;
        uint64_t gen = 0;
        bool valid = false;
    } rkey;
    size_t glu_cap = 0;
    void * glu = nullptr;            // gate/up sums of qmm_mul_mat_glu
    // the slots of the fused GEMV's K-slice tree: filled with kTreeEmpty when allocated, and
    // every launch leaves them so
    uint32_t * tree = nullptr;
    size_t tree_words = 0;
    // downgrades: ops that took a slower path than their weight type promises, counted per key
    // in fixed storage (recording one allocates nothing); keys past the table count as "other"
    struct Downgrade {
        char key[112];
        int64_t count;
    };
    static constexpr int kMaxDowngradeKeys = 48;
    Downgrade dg[kMaxDowngradeKeys];
    int n_dg = 0;
    int64_t dg_other = 0;
    // the activation scratch of qmm_mul_mat_noalloc on this context's device (a __device__
    // array of this file; its address comes from hipGetSymbolAddress at context creation)
    uint8_t * fixed_scratch = nullptr;
    // main-kernel timing (qmm_kernel_timing)
    bool ktime = false;
    bool ktime_markers = false;    // event records around the launch instead of dispatch stamps
    hipEvent_t ktime_stop = nullptr;   // marker mode: the stop event of the launch just made
    std::vector<hipEvent_t> kev;   // pairs
    size_t kev_used = 0;
    // HIP-graph capture of the stream (qmm_capture_begin/end): ops allocate nothing and record
    // no timing events meanwhile; a failure while capturing makes qmm_capture_end fail
    bool capturing = false;
    bool capture_failed = false;
    // bumped whenever a scratch buffer the kernels read is freed for a larger one: a graph
    // captured before then points at freed memory and is refused (qmm_graph_launch)
    uint64_t scratch_gen = 0;
    int capture_code = 0;          // the first failure while capturing, and its reason
    std::string capture_err;
};

// an instantiated capture (qmm_capture_end)
struct qmm_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int device = 0;
    const qmm_ctx * ctx = nullptr;   // the context captured from, and its scratch generation then
    uint64_t scratch_gen = 0;
};

namespace {

int fail(qmm_ctx * ctx, int code, const char * fmt, ...) {
    if (ctx) {
        const bool first_in_capture = ctx->capturing && !ctx->capture_failed;
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        ctx->err = buf;
        if (first_in_capture) {
            ctx->capture_failed = true;
            ctx->capture_code = code;
            ctx->capture_err = buf;
        }
    }
    return code;
}

#define QMM_HIP(ctx, expr)                                                                        \
    do {                                                                                          \
        const hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess) return fail((ctx), QMM_ERR_DEVICE, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

bool is_quant(int type) { return type_layout(type) != nullptr; }

size_t plain_elem(int type) {
    switch (type) {
        case QMM_TYPE_F32: return 4;
        case QMM_TYPE_F16: return 2;
        case QMM_TYPE_I32: return 4;
        default: return 0;
    }
}

int64_t nelements(const int64_t ne[4]) { return ne[0] * ne[1] * ne[2] * ne[3]; }

bool contiguous(const qmm_tensor * t) {
    const TypeLayout * L = type_layout(t->type);
    size_t s = L ? (size_t)L->bytes : plain_elem(t->type);
    int64_t n0 = L ? t->ne[0] / L->blck : t->ne[0];
    if (t->nb[0] != s) return false;
    size_t expect = s * (size_t)n0;
    for (int i = 1; i < 4; ++i) {
        if (t->ne[i] > 1 && t->nb[i] != expect) return false;
        expect *= (size_t)t->ne[i];
    }
    return true;
}

static bool why(char * reason, size_t len, const char * msg) {
    if (reason && len) snprintf(reason, len, "%s", msg);
    return false;
}

// the tensor that owns a quantized tensor's device image (ggml keeps view_src a non-view)
static const qmm_tensor * base_of(const qmm_tensor * t) { return t->view_src ? t->view_src : t; }

// ggml_nbytes: the bytes from a tensor's first to past its last element, strides as given
static size_t view_nbytes(const qmm_tensor * t) {
    size_t bb = 0;
    const int bl = qmm_type_block(t->type, &bb);
    if (!bl || t->ne[0] % bl) return 0;
    size_t n = (size_t)(t->ne[0] / bl) * t->nb[0];
    for (int i = 1; i < 4; ++i) {
        if (t->ne[i] <= 0) return 0;
        n += (size_t)(t->ne[i] - 1) * t->nb[i];
    }
    return n;
}

// the last byte a tensor view touches lies inside its buffer
static bool span_ok(const qmm_tensor * t) {
    size_t last = 0;
    for (int i = 0; i < 4; ++i) {
        if (t->ne[i] <= 0) return false;
        last += (size_t)(t->ne[i] - 1) * t->nb[i];
    }
    return t->offs + last + t->nb[0] <= t->buffer->size;
}

// The device image the kernels read for a quantized tensor: its own, or the part of its
// base's image a view covers.  A view is taken when its matrices are whole matrices of the
// base (the reference's whole-slice rule, 0116-opencl-q3_K.patch:76-85) or, when every base
// matrix is whole 64-row tiles, whole tiles of it: then its rows sit in the base image at a
// tile boundary exactly as its own shape would lay them out.  `mem` also checks that the
// image lies in its buffer (off for shape-only queries).
static bool weight_image(const qmm_tensor * t, bool mem, WView * w, char * reason, size_t len) {
    const TypeLayout * L = type_layout(t->type);
    if (!L) return why(reason, len, "src0 type is not Q4_0/Q8_0/Q4_K/Q5_K/Q6_K/IQ4_NL/IQ4_XS");
    if (t->ne[0] % L->blck) return why(reason, len, "ne00 is not a multiple of the block size");
    if (!contiguous(t)) return why(reason, len, "src0 is not contiguous");
    const qmm_tensor * b = base_of(t);
    if (b != t && (b->view_src || b->type != t->type || b->ne[0] != t->ne[0] || !contiguous(b)))
        return why(reason, len, "src0 view: its base is not a contiguous tensor of its type and row length");
    ImageShape bs, vs;
    if (!image_shape(*L, b->ne, &bs) || !image_shape(*L, t->ne, &vs)) return why(reason, len, "src0 shape");
    if (b->offs % kPlaneAlign) return why(reason, len, "src0 offset is not a multiple of 256");
    if (mem) {
        if (!b->buffer) return why(reason, len, "src0 has no buffer");
        if (b->offs > b->buffer->size || bs.bytes > b->buffer->size - b->offs)
            return why(reason, len, "src0 image runs past its buffer");
    }
    const size_t row = (size_t)bs.bpr * (size_t)L->bytes, tile = (size_t)bs.G * (size_t)L->tg;
    const size_t voff = b == t ? 0 : t->view_offs;
    if (voff % row) return why(reason, len, "src0 view does not start on a row of its base");
    const int64_t R0 = (int64_t)(voff / row), rows = t->ne[1] * t->ne[2] * t->ne[3];
    if (R0 + rows > bs.M * bs.nmat) return why(reason, len, "src0 view runs past its base");
    size_t at;
    if (t->ne[1] == bs.M && R0 % bs.M == 0)
        at = (size_t)(R0 / bs.M) * (size_t)bs.ntiles * tile;                       // whole matrices
    else if (bs.M % kTileRows == 0 && t->ne[1] % kTileRows == 0 && R0 % kTileRows == 0)
        at = (size_t)(R0 / kTileRows) * tile;                                      // whole tiles
    else
        return why(reason, len, "src0 view is not whole matrices or whole 64-row tiles of its base");
    w->base = mem ? (const uint8_t *)b->buffer->ptr + b->offs + at : nullptr;
    w->M = vs.M;
    w->K = vs.K;
    w->bpr = vs.bpr;
    w->G = vs.G;
    w->ntiles = vs.ntiles;
    w->tg = L->tg;
    return true;
}

// activation scratch layout for ncols columns of ldk (K rounded up to 256):
// codes, scales, sums and (GEMM consumers) the scales again block-major with
// a row stride of ldT
size_t act_bytes(int vdt, int64_t ldk, int64_t ncols, bool dT, int64_t ldT, size_t * o_d, size_t * o_s, size_t * o_t,
                 size_t * o_b) {
    size_t off = align_up((size_t)(ldk * ncols), kPlaneAlign);
    *o_d = off;
    off = align_up(off + (size_t)(ncols * (ldk / act_block(vdt))) * 4, kPlaneAlign);
    *o_s = off;
    off = align_up(off + (size_t)(ncols * (ldk / act_sum_block(vdt))) * 2, kPlaneAlign);
    *o_t = off;
    if (dT) off = align_up(off + (size_t)((ldk / act_block(vdt)) * ldT) * 4, kPlaneAlign);
    *o_b = off;
    if (vdt == QMM_TYPE_Q8_K) off = align_up(off + (size_t)((ldk / 256) * ldT) * 16, kPlaneAlign);
    return off;
}

int ensure(qmm_ctx * ctx, void ** p, size_t * cap, size_t need) {
    if (need <= *cap) return QMM_OK;
    if (ctx->capturing)
        return fail(ctx, QMM_ERR_NOMEM, "capture: the op needs %zu bytes of scratch and the context has %zu; run it "
                                        "once outside a capture first", need, *cap);
    if (*p) {
        QMM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        QMM_HIP(ctx, hipFree(*p));
        *p = nullptr;
        *cap = 0;
        ctx->key.valid = false;
        ctx->scratch_gen++;
    }
    size_t sz = std::max(need, (size_t)(*cap * 3 / 2));
    QMM_HIP(ctx, hipMalloc(p, sz));
    *cap = sz;
    return QMM_OK;
}

// tree slots for a split fused GEMV: grown outside captures only, each new allocation filled
// with kTreeEmpty on the stream ahead of its first use
int ensure_tree(qmm_ctx * ctx, size_t words) {
    if (words <= ctx->tree_words) return QMM_OK;
    if (ctx->capturing)
        return fail(ctx, QMM_ERR_NOMEM, "capture: the op needs %zu words of tree slots and the context has %zu; run "
                                        "it once outside a capture first", words, ctx->tree_words);
    if (ctx->tree) {
        QMM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        QMM_HIP(ctx, hipFree(ctx->tree));
        ctx->tree = nullptr;
        ctx->tree_words = 0;
        ctx->scratch_gen++;
    }
    const size_t n = std::max(words, ctx->tree_words * 3 / 2);
    QMM_HIP(ctx, hipMalloc((void **)&ctx->tree, n * 4));
    QMM_HIP(ctx, hipMemsetD32Async((hipDeviceptr_t)ctx->tree, (int)kTreeEmpty, n, ctx->stream));
    ctx->tree_words = n;
    return QMM_OK;
}

F32Cols f32_cols(const qmm_tensor * t) {
    F32Cols c;
    c.base = (const char *)t->buffer->ptr + t->offs;
    c.ne1 = t->ne[1];
    c.ne2 = t->ne[2];
    c.nb1 = t->nb[1];
    c.nb2 = t->nb[2];
    c.nb3 = t->nb[3];
    return c;
}

bool same_key(const qmm_ctx * ctx, int vdt, const qmm_tensor * src1, bool dT, bool tiled) {
    const auto & k = ctx->key;
    return k.valid && k.gen == ctx->graph_gen && k.buf == src1->buffer && k.offs == src1->offs && k.vdt == vdt &&
           k.tiled == tiled && (k.dT || !dT) && !memcmp(k.ne, src1->ne, sizeof(k.ne)) &&
           !memcmp(k.nb, src1->nb, sizeof(k.nb));
}

// Quantize src1 (all its columns) with the vec_dot type of `type`, reusing
// the previous result inside one graph when src1 is the same tensor.
// a MUL_MAT_ID route whose launch joins the activation quantization's (the two are independent)
struct PendingRoute {
    RouteArgs r;
    int32_t * scratch;
    GemvTask * tasks;              // GEMV tasks, or
    int32_t * ntasks;
    GemmUnit * units = nullptr;    // the grouped GEMM's 64-column units (then tasks is unused)
};

// quantize src1 for the vec_dot type of `type` (skipped when this graph already did); with
// pr, the route runs in the same launch (or alone when the quantization is skipped)
// Device memory the activations go to instead of the context's scratch: nothing is allocated
// and the graph's activation cache is neither read nor written.
struct FixedAct {
    uint8_t * base;
    size_t cap;
};

int quantize_src1(qmm_ctx * ctx, int type, const qmm_tensor * src1, bool dT, ActBuf * out, const ZeroJob * z = nullptr,
                  const PendingRoute * pr = nullptr, const FixedAct * fixed = nullptr) {
    const int vdt = vec_dot_type(type);
    const int64_t K = src1->ne[0], ncols = src1->ne[1] * src1->ne[2] * src1->ne[3];
    auto & k = ctx->key;
    if (pr && z) return fail(ctx, QMM_ERR_INVALID, "internal: a route launch with dst zeroing");
    if (!fixed && ctx->in_graph && same_key(ctx, vdt, src1, dT, false)) {
        *out = ctx->cached;
        if (z) QMM_HIP(ctx, launch_quantize(f32_cols(src1), K, 0, ctx->cached, z, ctx->stream));   // zeroing only
        if (pr && pr->units) QMM_HIP(ctx, launch_route(pr->r, pr->scratch, pr->units, pr->ntasks, ctx->stream));
        else if (pr) QMM_HIP(ctx, launch_route(pr->r, pr->scratch, pr->tasks, pr->ntasks, ctx->stream));
        return QMM_OK;
    }
    size_t od, os, ot, ob;
    const int64_t ldk = (K + 255) / 256 * 256;
    const int64_t ldT = (ncols + 3) / 4 * 4 + 64;    // the GEMM reads up to 63 columns past the last
    const size_t need = act_bytes(vdt, ldk, ncols, dT, ldT, &od, &os, &ot, &ob);
    if (fixed && need > fixed->cap)
        return fail(ctx, QMM_ERR_NOMEM, "the activations of src1 [%lld, %lld] need %zu bytes of scratch; at most %zu",
                    (long long)K, (long long)ncols, need, fixed->cap);
    if (!fixed) {
        const int rc = ensure(ctx, &ctx->act, &ctx->act_cap, need);
        if (rc) return rc;
    }
    uint8_t * b = fixed ? fixed->base : (uint8_t *)ctx->act;
    ActBuf a;
    a.codes = (int8_t *)b;
    a.d = (float *)(b + od);
    a.sums = (int16_t *)(b + os);
    a.dT = dT ? (float *)(b + ot) : nullptr;
    a.bsp = vdt == QMM_TYPE_Q8_K ? (int8_t *)(b + ob) : nullptr;
    a.ldT = ldT;
    a.K = K;
    a.ldk = ldk;
    a.ncols = ncols;
    a.vdt = vdt;
    if (pr && pr->units)
        QMM_HIP(ctx, launch_quant_route(f32_cols(src1), K, ncols, a, pr->r, pr->scratch, pr->units, pr->ntasks, ctx->stream));
    else if (pr)
        QMM_HIP(ctx, launch_quant_route(f32_cols(src1), K, ncols, a, pr->r, pr->scratch, pr->tasks, pr->ntasks, ctx->stream));
    else QMM_HIP(ctx, launch_quantize(f32_cols(src1), K, ncols, a, z, ctx->stream));
    *out = a;
    if (fixed) return QMM_OK;
    k.buf = src1->buffer;
    k.offs = src1->offs;
    memcpy(k.ne, src1->ne, sizeof(k.ne));
    memcpy(k.nb, src1->nb, sizeof(k.nb));
    k.vdt = vdt;
    k.dT = dT;
    k.tiled = false;
    k.gen = ctx->graph_gen;
    k.valid = true;
    ctx->cached = a;
    return QMM_OK;
}

// Quantize src1 (the vec_dot type of `type`: q8_0, or q8_K for Q4_K) into the streaming GEMM's
// tiled layout for weights of G groups per row, reusing the previous result inside one graph
// when src1 is the same tensor.
int quantize_src1_tiled(qmm_ctx * ctx, int type, const qmm_tensor * src1, int64_t G, TiledAct * out,
                        const FixedAct * fixed = nullptr) {
    const int64_t K = src1->ne[0], N = src1->ne[1], nbatch = src1->ne[2] * src1->ne[3];
    const int vdt = vec_dot_type(type);
    auto & k = ctx->key;
    if (!fixed && ctx->in_graph && same_key(ctx, vdt, src1, false, true) && ctx->cached_tiled.nblk == G * 8) {
        *out = ctx->cached_tiled;
        return QMM_OK;
    }
    TiledAct t;
    t.nblk = G * 8;
    t.ntb = (N + 31) / 32;
    t.ntiles = t.ntb * nbatch;
    t.N = N;
    t.vdt = vdt;
    // q8_K: one scale per 8 blocks, and the split sub-block sums
    const bool kq = vdt == QMM_TYPE_Q8_K;
    const size_t oa = tiled_a_bytes(t.ntiles, t.nblk);
    const size_t od = tiled_d_bytes(t.ntiles, kq ? t.nblk / 8 : t.nblk);
    const size_t need = oa + od + (kq ? tiled_s_bytes(t.ntiles, t.nblk) : 0);
    if (fixed && need > fixed->cap)
        return fail(ctx, QMM_ERR_NOMEM, "the activations of src1 [%lld, %lld] need %zu bytes of scratch; at most %zu",
                    (long long)K, (long long)(N * nbatch), need, fixed->cap);
    if (!fixed) {
        const int rc = ensure(ctx, &ctx->act, &ctx->act_cap, need);
        if (rc) return rc;
    }
    uint8_t * b = fixed ? fixed->base : (uint8_t *)ctx->act;
    t.A = (int8_t *)b;
    t.D = (float *)(b + oa);
    t.S = kq ? (int8_t *)(b + oa + od) : nullptr;
    QMM_HIP(ctx, launch_quantize_tiled(f32_cols(src1), K, t, ctx->stream));
    *out = t;
    if (fixed) return QMM_OK;
    k.buf = src1->buffer;
    k.offs = src1->offs;
    memcpy(k.ne, src1->ne, sizeof(k.ne));
    memcpy(k.nb, src1->nb, sizeof(k.nb));
    k.vdt = vdt;
    k.dT = false;
    k.tiled = true;
    k.gen = ctx->graph_gen;
    k.valid = true;
    ctx->cached_tiled = t;
    return QMM_OK;
}

bool ranges_overlap(const qmm_tensor * a, const qmm_tensor * b) {
    if (!a || !b || a->buffer != b->buffer) return false;
    auto span = [](const qmm_tensor * t) {
        size_t last = 0;
        for (int i = 0; i < 4; ++i) last += (size_t)(t->ne[i] - 1) * t->nb[i];
        return last + t->nb[0];
    };
    const size_t a0 = a->offs, a1 = a->offs + span(a), b0 = b->offs, b1 = b->offs + span(b);
    return a0 < b1 && b0 < a1;
}

bool f32_shape(const qmm_tensor * t) { return t && t->type == QMM_TYPE_F32 && t->nb[0] == sizeof(float) && t->ne[0] > 0; }

bool check_f32(const qmm_tensor * t) {
    return t && t->buffer && t->type == QMM_TYPE_F32 && t->nb[0] == sizeof(float) && t->ne[0] > 0;
}

// event pair stamped by the main kernel of an op when timing is on (null otherwise)
int ktime_pair(qmm_ctx * ctx, KTime * kt, const KTime ** out) {
    *out = nullptr;
    if (!ctx->ktime || ctx->capturing) return QMM_OK;
    if (ctx->kev_used + 2 > ctx->kev.size()) {
        for (int i = 0; i < 64; ++i) {
            hipEvent_t e;
            QMM_HIP(ctx, hipEventCreate(&e));
            ctx->kev.push_back(e);
        }
    }
    kt->start = ctx->kev[ctx->kev_used];
    kt->stop = ctx->kev[ctx->kev_used + 1];
    ctx->kev_used += 2;
    if (ctx->ktime_markers) {                                     // the caller launches next
        QMM_HIP(ctx, hipEventRecord(kt->start, ctx->stream));
        ctx->ktime_stop = kt->stop;
        return QMM_OK;
    }
    *out = kt;
    return QMM_OK;
}

// after the main kernel's launch: in marker mode, the stop event
int ktime_done(qmm_ctx * ctx) {
    if (ctx->ktime_stop) {
        const hipEvent_t e = ctx->ktime_stop;
        ctx->ktime_stop = nullptr;
        QMM_HIP(ctx, hipEventRecord(e, ctx->stream));
    }
    return QMM_OK;
}

const char * type_name(int type) {
    switch (type) {
        case QMM_TYPE_Q4_0: return "Q4_0";
        case QMM_TYPE_Q8_0: return "Q8_0";
        case QMM_TYPE_Q4_K: return "Q4_K";
        case QMM_TYPE_Q5_K: return "Q5_K";
        case QMM_TYPE_Q6_K: return "Q6_K";
        case QMM_TYPE_IQ4_NL: return "IQ4_NL";
        case QMM_TYPE_IQ4_XS: return "IQ4_XS";
        case QMM_TYPE_F32: return "F32";
        case QMM_TYPE_F16: return "F16";
        default: return "?";
    }
}

// column counts in the buckets the downgrade keys use (a key holds no per-request value)
const char * cols_bucket(int64_t n) {
    return n <= 1 ? "1" : n <= 8 ? "2-8" : n <= 16 ? "9-16" : n <= 32 ? "17-32" : n <= 128 ? "33-128" : "129+";
}

// one downgrade under a key (the reference's ggml_cl_downgrade, 0100-...patch:44-66): counted per
// key; the first of a key is logged to stderr when QMM_DOWNGRADE_LOG is set
void note_downgrade(qmm_ctx * ctx, const char * fmt, ...) {
    char key[sizeof(ctx->dg[0].key)];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(key, sizeof(key), fmt, ap);
    va_end(ap);
    for (int i = 0; i < ctx->n_dg; ++i) {
        if (!strcmp(ctx->dg[i].key, key)) {
            ctx->dg[i].count++;
            return;
        }
    }
    if (ctx->n_dg == qmm_ctx::kMaxDowngradeKeys) {
        ctx->dg_other++;
        return;
    }
    memcpy(ctx->dg[ctx->n_dg].key, key, sizeof(key));
    ctx->dg[ctx->n_dg++].count = 1;
    if (getenv("QMM_DOWNGRADE_LOG")) fprintf(stderr, "DOWNGRADE src=qmm %s\n", key);
}

// the device address of `scratch` on `device`, which must be current: looked up once per
// device and kept (every context on that device shares the array)
std::mutex g_scratch_mu;
constexpr int kMaxDevices = 64;
uint8_t * g_scratch_ptr[kMaxDevices] = {};

hipError_t scratch_address(int device, uint8_t ** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    if (!g_scratch_ptr[device]) {
        void * p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[device] = (uint8_t *)p;
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

}  // namespace

// ---------------------------------------------------------------------------
extern "C" {

int qmm_ctx_create(int device, qmm_ctx ** out) {
    if (!out) return QMM_ERR_INVALID;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return QMM_ERR_DEVICE;
    qmm_ctx * ctx = new qmm_ctx();
    ctx->device = device;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&ctx->ev0) != hipSuccess || hipEventCreate(&ctx->ev1) != hipSuccess ||
        hipMalloc(&ctx->sink, kSinkBytes) != hipSuccess || hipMemsetAsync(ctx->sink, 0, kSinkBytes, ctx->stream) != hipSuccess ||
        hipMalloc(&ctx->dflags, 256) != hipSuccess || hipMemsetAsync(ctx->dflags, 0, 256, ctx->stream) != hipSuccess ||
        hipHostMalloc(&ctx->hflags, 256, hipHostMallocDefault) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess || scratch_address(device, &ctx->fixed_scratch) != hipSuccess) {
        qmm_ctx_free(ctx);
        return QMM_ERR_DEVICE;
    }
    *out = ctx;
    return QMM_OK;
}

// teardown: errors here have no caller to go to (void API, as ggml's free)
void qmm_ctx_free(qmm_ctx * ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->capturing) {                            // a capture left open: end it, drop its graph
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(ctx->stream, &g);
        if (g) (void)hipGraphDestroy(g);
        ctx->capturing = false;
    }
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->act) (void)hipFree(ctx->act);
    if (ctx->route) (void)hipFree(ctx->route);
    if (ctx->glu) (void)hipFree(ctx->glu);
    if (ctx->tree) (void)hipFree(ctx->tree);
    if (ctx->sink) (void)hipFree(ctx->sink);
    if (ctx->dflags) (void)hipFree(ctx->dflags);
    if (ctx->hflags) (void)hipHostFree(ctx->hflags);
    for (hipEvent_t e : ctx->kev) (void)hipEventDestroy(e);
    if (ctx->ev0) (void)hipEventDestroy(ctx->ev0);
    if (ctx->ev1) (void)hipEventDestroy(ctx->ev1);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

const char * qmm_last_error(qmm_ctx * ctx) { return ctx ? ctx->err.c_str() : "no context"; }
const char * qmm_last_path(qmm_ctx * ctx) { return ctx ? ctx->path.c_str() : "none"; }

int qmm_buffer_alloc(qmm_ctx * ctx, size_t size, qmm_buffer ** out) {
    if (!ctx || !out) return QMM_ERR_INVALID;
    *out = nullptr;
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    qmm_buffer * b = new qmm_buffer();
    const hipError_t e = hipMalloc(&b->ptr, std::max<size_t>(size, 256));
    if (e != hipSuccess) {
        delete b;
        return fail(ctx, QMM_ERR_NOMEM, "hipMalloc(%zu): %s", size, hipGetErrorString(e));
    }
    b->size = size;
    *out = b;
    return QMM_OK;
}

void qmm_buffer_free(qmm_ctx * ctx, qmm_buffer * buf) {
    if (!buf) return;
    if (ctx && ctx->capturing) {                      // (it synchronizes the stream: refused, buffer kept)
        (void)fail(ctx, QMM_ERR_INVALID, "buffer_free: not while capturing (it synchronizes the stream)");
        return;
    }
    if (ctx) {
        (void)hipStreamSynchronize(ctx->stream);
        if (ctx->key.buf == buf) ctx->key.valid = false;
    }
    (void)hipFree(buf->ptr);
    delete buf;
}

size_t qmm_buffer_size(const qmm_buffer * buf) { return buf ? buf->size : 0; }
void * qmm_buffer_base(const qmm_buffer * buf) { return buf ? buf->ptr : nullptr; }

int qmm_type_block(int32_t type, size_t * block_bytes) {
    if (const TypeLayout * L = type_layout(type)) {
        if (block_bytes) *block_bytes = (size_t)L->bytes;
        return L->blck;
    }
    const size_t e = plain_elem(type);
    if (!e) return 0;
    if (block_bytes) *block_bytes = e;
    return 1;
}

size_t qmm_tensor_nbytes(int32_t type, const int64_t ne[4]) {
    size_t bb = 0;
    const int bl = qmm_type_block(type, &bb);
    if (!bl || ne[0] % bl) return 0;
    return (size_t)(nelements(ne) / bl) * bb;
}

size_t qmm_tensor_alloc_size(int32_t type, const int64_t ne[4]) {
    const TypeLayout * L = type_layout(type);
    if (!L) return qmm_tensor_nbytes(type, ne);
    ImageShape sh;
    if (!image_shape(*L, ne, &sh)) return 0;
    return sh.bytes;
}

// Quantized tensor IO: GGUF blocks [b0, b0 + nb) <-> the device image, staged
// through host memory a run of whole tiles at a time.  A write that leaves
// some row of a run untouched reads the run first (read-modify-write).
static int quant_io(qmm_ctx * ctx, const TypeLayout & L, const ImageShape & sh, uint8_t * dev, uint8_t * host,
                    int64_t b0, int64_t nb, bool write) {
    if (nb <= 0) return QMM_OK;
    const int64_t R0 = b0 / sh.bpr, R1 = (b0 + nb - 1) / sh.bpr + 1;
    const int64_t Ta = tile_of_row(sh, R0), Tb = tile_of_row(sh, R1 - 1) + 1;
    const size_t tile_bytes = (size_t)sh.G * (size_t)L.tg;
    const int64_t run = std::max<int64_t>(1, (int64_t)((64u << 20) / tile_bytes));
    std::vector<uint8_t> stage;
    for (int64_t T0 = Ta; T0 < Tb; T0 += run) {
        const int64_t T1 = std::min(Tb, T0 + run);
        int64_t rowA, rowB, dummy;
        tile_rows(sh, T0, &rowA, &dummy);
        tile_rows(sh, T1 - 1, &dummy, &rowB);
        const int64_t blkA = std::max(b0, rowA * sh.bpr), blkB = std::min(b0 + nb, rowB * sh.bpr);
        const size_t bytes = (size_t)(T1 - T0) * tile_bytes;
        uint8_t * d = dev + (size_t)T0 * tile_bytes;
        stage.assign(bytes, 0);
        const bool full = blkA == rowA * sh.bpr && blkB == rowB * sh.bpr;
        if (!write || !full) {
            QMM_HIP(ctx, hipMemcpyAsync(stage.data(), d, bytes, hipMemcpyDeviceToHost, ctx->stream));
            QMM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        }
        if (write) {
            pack_blocks(L, sh, host + (size_t)(blkA - b0) * L.bytes, blkA, blkB - blkA, stage.data(), T0);
            if (!full)
                for (int64_t R = blkA / sh.bpr; R <= (blkB - 1) / sh.bpr; ++R) zero_row_padding(L, sh, R, stage.data(), T0);
            QMM_HIP(ctx, hipMemcpyAsync(d, stage.data(), bytes, hipMemcpyHostToDevice, ctx->stream));
            QMM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        } else {
            unpack_blocks(L, sh, stage.data(), T0, blkA, blkB - blkA, host + (size_t)(blkA - b0) * L.bytes);
        }
    }
    return QMM_OK;
}

// GGUF bytes [lo, lo + size) of a quantized base: the whole blocks straight through quant_io,
// a block that either end of the range cuts read first and patched (read-modify-write), the
// reference's any-range rule (0116-opencl-q3_K.patch:113-133)
static int quant_range_io(qmm_ctx * ctx, const TypeLayout & L, const ImageShape & sh, uint8_t * dev, uint8_t * host,
                          size_t lo, size_t size, bool write) {
    const size_t bb = (size_t)L.bytes, hi = lo + size;
    if (lo % bb == 0 && hi % bb == 0)
        return quant_io(ctx, L, sh, dev, host, (int64_t)(lo / bb), (int64_t)(size / bb), write);
    std::vector<uint8_t> blk(bb);
    // the end blocks of the range (one when it lies inside a block); those it covers in part
    const int64_t first = (int64_t)(lo / bb), last = (int64_t)((hi - 1) / bb);
    for (int64_t c = first; c <= last; c += std::max<int64_t>(1, last - first)) {
        const size_t b0 = (size_t)c * bb, a = std::max(lo, b0), e = std::min(hi, b0 + bb);
        if (a == b0 && e == b0 + bb) continue;              // whole: goes with the middle
        int rc = quant_io(ctx, L, sh, dev, blk.data(), c, 1, false);
        if (rc) return rc;
        if (write) {
            memcpy(blk.data() + (a - b0), host + (a - lo), e - a);
            if ((rc = quant_io(ctx, L, sh, dev, blk.data(), c, 1, true))) return rc;
        } else {
            memcpy(host + (a - lo), blk.data() + (a - b0), e - a);
        }
    }
    const size_t w0 = (lo + bb - 1) / bb, w1 = hi / bb;    // blocks wholly inside the range
    if (w0 < w1) return quant_io(ctx, L, sh, dev, host + (w0 * bb - lo), (int64_t)w0, (int64_t)(w1 - w0), write);
    return QMM_OK;
}

// set_tensor / get_tensor (P02:1556-1790): bytes [offset, offset + size) of the tensor as
// ggml addresses them, data + offset, within ggml_nbytes.  A quantized view moves its base's
// bytes at view_offs + offset; the base's shape lays them out (0116-opencl-q3_K.patch:56-59).
static int tensor_io(qmm_ctx * ctx, const qmm_tensor * t, void * host, size_t offset, size_t size, bool write) {
    if (!ctx || !t || (!host && size)) return fail(ctx, QMM_ERR_INVALID, "tensor io: null argument");
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    const size_t span = view_nbytes(t);
    if (!span) return fail(ctx, QMM_ERR_INVALID, "tensor io: type %d / shape has no GGUF size", t->type);
    if (offset > span || size > span - offset) return fail(ctx, QMM_ERR_INVALID, "tensor io: range past the tensor");
    const TypeLayout * L = type_layout(t->type);
    const qmm_tensor * b = L ? base_of(t) : t;
    if (!b->buffer) return fail(ctx, QMM_ERR_INVALID, "tensor io: no buffer");
    if (write) ctx->key.valid = ctx->rkey.valid = false;
    if (!L) {   // the device bytes are the plain bytes
        if (t->offs > b->buffer->size || offset + size > b->buffer->size - t->offs)
            return fail(ctx, QMM_ERR_INVALID, "tensor io: range past its buffer");
        uint8_t * dev = (uint8_t *)b->buffer->ptr + t->offs + offset;
        if (!size) return QMM_OK;
        if (write) QMM_HIP(ctx, hipMemcpyAsync(dev, host, size, hipMemcpyHostToDevice, ctx->stream));
        else QMM_HIP(ctx, hipMemcpyAsync(host, dev, size, hipMemcpyDeviceToHost, ctx->stream));
        QMM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        return QMM_OK;
    }
    if (b != t && (b->view_src || b->type != t->type))
        return fail(ctx, QMM_ERR_INVALID, "tensor io: view_src is a view or of another type");
    if (!contiguous(b)) return fail(ctx, QMM_ERR_INVALID, "tensor io: the base tensor is not contiguous");
    const size_t total = qmm_tensor_nbytes(b->type, b->ne);
    const size_t lo = (b == t ? 0 : t->view_offs) + offset;
    if (lo > total || size > total - lo) return fail(ctx, QMM_ERR_INVALID, "tensor io: range past the view's base");
    const size_t alloc = qmm_tensor_alloc_size(b->type, b->ne);
    if (b->offs > b->buffer->size || alloc > b->buffer->size - b->offs)
        return fail(ctx, QMM_ERR_INVALID, "tensor io: tensor past its buffer");
    if (!size) return QMM_OK;
    ImageShape sh;
    image_shape(*L, b->ne, &sh);
    return quant_range_io(ctx, *L, sh, (uint8_t *)b->buffer->ptr + b->offs, (uint8_t *)host, lo, size, write);
}

int qmm_tensor_pack(int32_t type, const int64_t ne[4], const void * gguf, void * image, size_t image_size) {
    const TypeLayout * L = type_layout(type);
    ImageShape sh;
    if (!L || !gguf || !image || !image_shape(*L, ne, &sh) || image_size < sh.bytes) return QMM_ERR_INVALID;
    memset(image, 0, sh.bytes);
    pack_blocks(*L, sh, (const uint8_t *)gguf, 0, sh.nmat * sh.M * sh.bpr, (uint8_t *)image, 0);
    return QMM_OK;
}

int qmm_tensor_unpack(int32_t type, const int64_t ne[4], const void * image, void * gguf, size_t gguf_size) {
    const TypeLayout * L = type_layout(type);
    ImageShape sh;
    if (!L || !gguf || !image || !image_shape(*L, ne, &sh)) return QMM_ERR_INVALID;
    const int64_t nblk = sh.nmat * sh.M * sh.bpr;
    if (gguf_size < (size_t)nblk * (size_t)L->bytes) return QMM_ERR_INVALID;
    unpack_blocks(*L, sh, (const uint8_t *)image, 0, 0, nblk, (uint8_t *)gguf);
    return QMM_OK;
}

int qmm_tensor_set(qmm_ctx * ctx, const qmm_tensor * t, const void * data, size_t offset, size_t size) {
    if (ctx && ctx->capturing) return fail(ctx, QMM_ERR_INVALID, "tensor_set: not while capturing (it synchronizes the stream)");
    return tensor_io(ctx, t, const_cast<void *>(data), offset, size, true);
}

int qmm_tensor_get(qmm_ctx * ctx, const qmm_tensor * t, void * data, size_t offset, size_t size) {
    if (ctx && ctx->capturing) return fail(ctx, QMM_ERR_INVALID, "tensor_get: not while capturing (it synchronizes the stream)");
    return tensor_io(ctx, t, data, offset, size, false);
}

int qmm_buffer_copy(qmm_ctx * ctx, qmm_buffer * dst, size_t dst_off, const qmm_buffer * src, size_t src_off, size_t size) {
    if (!ctx || !dst || !src || dst_off + size > dst->size || src_off + size > src->size)
        return fail(ctx, QMM_ERR_INVALID, "buffer copy out of range");
    QMM_HIP(ctx, hipMemcpyAsync((uint8_t *)dst->ptr + dst_off, (const uint8_t *)src->ptr + src_off, size,
                                hipMemcpyDeviceToDevice, ctx->stream));
    return QMM_OK;
}

// ---- validation ------------------------------------------------------------

// `mem`: also check that every operand lies inside its buffer (off for shape-only queries)
static bool mul_mat_ok(const qmm_tensor * s0, const qmm_tensor * s1, const qmm_tensor * d, bool mem, WView * w,
                       char * reason, size_t len) {
    if (!s0 || !s1 || !d) return why(reason, len, "null tensor");
    if (!weight_image(s0, mem, w, reason, len)) return false;
    if (!f32_shape(s1) || !f32_shape(d)) return why(reason, len, "src1/dst must be f32 with nb[0] == 4");
    if (mem && (!s1->buffer || !d->buffer)) return why(reason, len, "src1/dst has no buffer");
    if (mem && (!span_ok(s1) || !span_ok(d))) return why(reason, len, "src1/dst runs past its buffer");
    if (s1->ne[0] != s0->ne[0]) return why(reason, len, "src1 ne0 != src0 ne0");
    if (s1->ne[0] % 256 && vec_dot_type(s0->type) == QMM_TYPE_Q8_K) return why(reason, len, "K is not a multiple of 256");
    if (s0->ne[2] <= 0 || s0->ne[3] <= 0 || s1->ne[2] % s0->ne[2] || s1->ne[3] % s0->ne[3])
        return why(reason, len, "src1 dims 2/3 do not broadcast src0");
    if (d->ne[0] != s0->ne[1] || d->ne[1] != s1->ne[1] || d->ne[2] != s1->ne[2] || d->ne[3] != s1->ne[3])
        return why(reason, len, "dst shape is not [M, N, ne12, ne13]");
    if (d->nb[1] % 4 || d->nb[2] % 4 || d->nb[3] % 4) return why(reason, len, "dst strides are not whole floats");
    if (s1->nb[1] % 4 || s1->nb[2] % 4 || s1->nb[3] % 4 || s1->offs % 4) return why(reason, len, "src1 strides are not whole floats");
    return true;
}

static bool mul_mat_id_ok(const qmm_tensor * s0, const qmm_tensor * s1, const qmm_tensor * ids, const qmm_tensor * d,
                          bool mem, WView * w, char * reason, size_t len) {
    if (!s0 || !s1 || !ids || !d) return why(reason, len, "null tensor");
    if (!weight_image(s0, mem, w, reason, len)) return false;
    if (s0->ne[3] != 1) return why(reason, len, "src0 must be [K, M, n_as]");
    if (!f32_shape(s1) || !f32_shape(d)) return why(reason, len, "src1/dst must be f32 with nb[0] == 4");
    if (ids->type != QMM_TYPE_I32 || ids->nb[0] != 4) return why(reason, len, "ids must be i32");
    if (mem && (!s1->buffer || !d->buffer || !ids->buffer)) return why(reason, len, "src1/ids/dst has no buffer");
    if (mem && (!span_ok(s1) || !span_ok(d) || !span_ok(ids))) return why(reason, len, "src1/ids/dst runs past its buffer");
    if (s1->ne[0] != s0->ne[0]) return why(reason, len, "src1 ne0 != src0 ne0");
    if (s1->ne[0] % 256 && vec_dot_type(s0->type) == QMM_TYPE_Q8_K) return why(reason, len, "K is not a multiple of 256");
    const int64_t n_used = ids->ne[0], T = ids->ne[1];
    if (s1->ne[2] != T || s1->ne[3] != 1) return why(reason, len, "src1 must be [K, ne11, T]");
    if (s1->ne[1] != 1 && s1->ne[1] != n_used) return why(reason, len, "src1 ne11 must be 1 or n_used");
    if (d->ne[0] != s0->ne[1] || d->ne[1] != n_used || d->ne[2] != T) return why(reason, len, "dst must be [M, n_used, T]");
    if (s0->ne[2] > 8192) return why(reason, len, "more than 8192 experts");
    if (d->nb[1] % 4 || d->nb[2] % 4) return why(reason, len, "dst strides are not whole floats");
    if (s1->nb[1] % 4 || s1->nb[2] % 4 || s1->offs % 4) return why(reason, len, "src1 strides are not whole floats");
    return true;
}

// shapes, types and views only: ggml's scheduler asks before the activations have memory
int qmm_supports_op(qmm_ctx *, int32_t op, const qmm_tensor * src0, const qmm_tensor * src1, const qmm_tensor * ids,
                    const qmm_tensor * dst, char * reason, size_t reason_len) {
    WView w;
    if (op == QMM_OP_MUL_MAT) return mul_mat_ok(src0, src1, dst, false, &w, reason, reason_len) ? 1 : 0;
    if (op == QMM_OP_MUL_MAT_ID) return mul_mat_id_ok(src0, src1, ids, dst, false, &w, reason, reason_len) ? 1 : 0;
    why(reason, reason_len, "op is not MUL_MAT or MUL_MAT_ID");
    return 0;
}

// ---- ops ---------------------------------------------------------------------

// few columns (this many and up to 32 per weight pass) on the MFMA GEMV; QMM_GEMV_MMA_MIN overrides
static int gemv_mma_min_cols() {
    const char * e = getenv("QMM_GEMV_MMA_MIN");
    return e ? std::max(2, atoi(e)) : 3;
}

// columns at or above which MUL_MAT may go to the GEMM instead of the GEMV (32 columns per
// weight pass on the MFMA GEMV, 8 on v_dot4): within one MFMA GEMV pass the GEMV won every
// measured shape (Q4_K 17408 x 5120 at 24-32: 25-29 against 30 us); past it use_gemm_for
// weighs the launch.  QMM_GEMM_MIN_COLS overrides.
static int64_t gemm_min_cols(int type) {
    const char * e = getenv("QMM_GEMM_MIN_COLS");
    if (e) return std::max<int64_t>(1, atoll(e));
    // (past one pass of the few-column MFMA GEMV; Q5_K, which has no MFMA GEMV, from 16: its
    // v_dot4 GEMV takes 8 columns a pass; use_gemm_for decides from there)
    return gemv_mma_supported(type) ? kMmaMaxCols + 1 : 16;
}

// MUL_MAT on the GEMM: from gemm_min_cols, when the streaming GEMM's launch gives every SIMD a
// wave (rows x column units x K slices >= 1024); with fewer (down to 512) when the GEMV would
// stream enough weight bytes over its passes (32 columns a pass on the MFMA GEMV, 8 on v_dot4):
// 90 MB.  Q6_K, whose GEMM costs more per MAC, needs 400 MB at any wave count below 256 columns.
// Else the GEMV's tasks, which split K over work-groups.  Measured (op us, GEMV / GEMM): Q4_K 17408 x 5120 at N = 40-64 44.7-50.8 / 31,
// 12288 x 5120 at 48 30.0 / 30.0, 5120 x 6144 at 48-64 22-24 / 32-33; Q6_K 5120 x 17408 at 128
// 96 / 116, at 192 141 / 122, the 151936-row head at 64 446 / 272; IQ4_XS 4096 x 14336 at 48-64
// 35-38 / 73; Q5_K 17408 x 5120 at 16-48 62-135 / 34-36; config 3's shared expert (Q4_K 512 x
// 2048, N = 256) 30.4 / 42.8.  QMM_GEMM_MIN_COLS, when set, decides alone.
static bool use_gemm_for(int type, const WView & w, int64_t N, int64_t nbatch) {
    if (N < gemm_min_cols(type)) return false;
    if (getenv("QMM_GEMM_MIN_COLS")) return true;
    G3Shape sh;
    if (!gemm3_shape(type, w, N, nbatch, &sh)) return true;      // (the shared-tile GEMM)
    const int64_t waves = sh.mbn * sh.nbn * nbatch * sh.U * sh.KS;
    const int64_t per = gemv_mma_supported(type) ? kMmaMaxCols : 8;
    const double passes = (double)((N + per - 1) / per);
    const double bytes = (double)(w.ntiles * w.G) * (double)w.tg * (double)nbatch;
    if (type == QMM_TYPE_Q6_K && N < 256) return waves >= 512 && passes >= 2 && passes * bytes >= 400e6;
    if (waves >= 1024) return true;
    return waves >= 512 && passes >= 2 && passes * bytes >= 90e6;
}

// columns per GEMV task: up to 32 on the MFMA kernel (the rows of its A operand), 8 on v_dot4,
// spread evenly over the fewest weight passes
static int gemv_task_cols(int type, int64_t N) {
    const int64_t cap = gemv_mma_supported(type) && N >= gemv_mma_min_cols() ? kMmaMaxCols : kMaxTaskCols;
    const int64_t passes = (N + cap - 1) / cap;
    return (int)((N + passes - 1) / passes);
}

// The fused-quantization GEMV (k_gemv_fq, no pre-pass launch).  MUL_MAT_ID of few tokens takes
// it (its pairs need no route launch: 13.3 -> 6.0 us per op at config 3's T = 1).  Dense
// products do not by default: with K split only among the waves of a work-group the chip runs
// unbalanced (17408 x 5120 Q4_K: 272 work-groups of 10 waves on 256 CUs, kernel 15.8 us against
// the split-K kernel's 12.7 us, whose pre-pass costs the op 0.8 us); QMM_GEMV_FQ_MIN_WAVES = n
// takes it for 1-2 columns when its work-groups give the chip n waves or more.
// QMM_GEMV_FUSED=0 switches the kernel off everywhere.
static bool fused_on() {
    const char * e = getenv("QMM_GEMV_FUSED");
    return !e || atoi(e) != 0;
}
static int64_t fused_min_waves() {
    const char * e = getenv("QMM_GEMV_FQ_MIN_WAVES");
    return e ? atoll(e) : INT64_MAX;
}
// MUL_MAT_ID below this many tokens reads its ids per (slot, token) pair in the GEMV (no route;
// the reference's per-pair matvec below 16 tokens, P01:1189-1192); QMM_MOE_DIRECT_T overrides
static int64_t moe_direct_tokens() {
    const char * e = getenv("QMM_MOE_DIRECT_T");
    return e ? atoll(e) : 16;
}

// Small dense products are the exception: at most 8 groups along K (one per wave) and 512
// tile-groups in all, the op is launch latency and one launch beats two (config 3's shared
// expert, N = 1: gate + up + SwiGLU 512 x 2048 9.1 -> 6.4 us, down 2048 x 512 6.8 -> 4.4 us;
// at 16 groups the fused kernel lost, Q4_0 2048 x 4096 7.5 against 6.5 us).
// QMM_GEMV_FQ_SMALL_TG sets the tile-group bound (0: never).
static int64_t fused_small_tgroups() {
    const char * e = getenv("QMM_GEMV_FQ_SMALL_TG");
    return e ? atoll(e) : 512;
}

// Dense products of 1-2 columns may also split K over work-groups of the fused kernel (its
// K-slice tree): one launch instead of the pre-pass and the GEMV.  Measured per op (bench,
// one box): one column of every type gains or ties (config 2's Q4_K 17408 x 5120 12.6 ->
// 11.6 us, Q5_K 14.7 -> 13.8, config 4's Q8_0 14.3 -> 13.9, Q4_0 4096 x 4096 7.0-8.9 -> 6.0; the
// IQ4 types within 1 %; Q6_K, two stages a group requested together, 16.6 -> 16.4 us and the
// output head 99.9 -> 99.2); two columns on large images lose (Q6_K 5120 x 17408 18.8 -> 20.3,
// Q8_0 14336 x 4096 15.3 -> 15.7, IQ4_XS 13.0-13.5 -> 14.2; with 8 waves a work-group Q8_0 gains
// at two columns too, 15.5 -> 14.8 us, while IQ4_XS ties and Q4_K loses 2-3 %).  So: one column
// of any type, two of Q8_0, and 1-2 columns of any type for images up to QMM_GEMV_FQS_MAX_KB
// (16 MiB) of one matrix;
// QMM_GEMV_FQS = 0 never, = 1 always;
// work-groups of QMM_GEMV_FQS_W waves with QMM_GEMV_FQS_SPW groups each (1): 4 waves (Q4_K 11.6
// us against 12.2-12.3 at 2, 5 and 8; Q5_K 14.1-14.2 against 15.7 at 8), 8 for Q8_0, whose
// 17 KB tile-groups run 2.5 % faster so (13.2 against 13.5 us on 14336 x 4096).
static int env_or(const char * name, int dflt) {
    const char * e = getenv(name);
    return e ? atoi(e) : dflt;
}
static bool fused_split_for(int type, const WView & w, int64_t N) {
    const int mode = env_or("QMM_GEMV_FQS", -1);
    if (mode == 0) return false;
    if (mode > 0) return true;
    if (N == 1) return true;
    if (N == 2 && type == QMM_TYPE_Q8_0) return true;            // (14336 x 4096: 15.5 -> 14.8 us)
    const int64_t image = w.ntiles * w.G * (int64_t)w.tg;
    return image <= (int64_t)env_or("QMM_GEMV_FQS_MAX_KB", 16384) * 1024;
}

// whether a dense product of N columns in nbatch batches takes the fused GEMV, and its plan;
// split: K may be split over work-groups (not where nothing may be allocated)
static bool fused_dense_plan(int type, const WView & w, int64_t N, int64_t nbatch, FusedPlan * fp, bool split) {
    if (!fused_on() || N < 1) return false;
    if (N > 2) {
        // 3-16 columns as 2-column tasks, on small products only (the bound above), where the
        // launches are the op: config 3's shared expert at T = 4 (Q4_K 512 x 2048 gate + up +
        // SwiGLU, 2048 x 512 down) ran as pre-pass + MFMA GEMV (+ GLU kernel), five launches
        if (N > 16 || !gemv_fused_plan(type, w, 2, (N + 1) / 2 * nbatch, gemv_fused_waves_target(), fp)) return false;
        return w.G <= 8 && fp->ntasks * w.ntiles * w.G <= fused_small_tgroups();
    }
    if (gemv_fused_plan(type, w, (int)N, nbatch, gemv_fused_waves_target(), fp)) {
        const int64_t tgroups = fp->ntasks * w.ntiles * w.G;
        if (w.G <= 8 && tgroups <= fused_small_tgroups()) return true;
        if (fp->ntasks * w.ntiles * fp->W >= fused_min_waves()) return true;
        // one column with each wave on one group and K whole in its work-group (no exchange
        // tree), given 3072 waves or more: 14336 x 4096 (3584 waves of 16-wave work-groups)
        // IQ4_XS 10.3-10.5 -> 9.64 us, IQ4_NL 9.8-10.0 -> 9.0, Q8_0 11.8-12.0 -> 11.36 against
        // the split form; Q4_0 4096 x 4096 (1024 waves) lost, 5.6 -> 6.5, and two groups a
        // wave lose everywhere (4096 x 14336: 10.7 -> 27 us)
        if (N == 1 && fp->spw == 1 && fp->ntasks * w.ntiles * fp->W >= 3072 && fused_min_waves() == INT64_MAX)
            return true;
    }
    return split && fused_split_for(type, w, N) &&
           gemv_fused_split_plan(type, w, (int)N, nbatch, env_or("QMM_GEMV_FQS_W", type == QMM_TYPE_Q8_0 ? 8 : 4),
                                 env_or("QMM_GEMV_FQS_SPW", 1), fp);
}
// whether a MUL_MAT_ID of T tokens with n_used ids each takes the fused GEMV's pairs, and its plan
static bool fused_id_plan(int type, const WView & w, int64_t n_used, int64_t T, FusedPlan * fp) {
    if (!fused_on() || T >= moe_direct_tokens()) return false;
    return gemv_fused_plan(type, w, 1, n_used * T, gemv_fused_waves_target(), fp);
}

int qmm_describe_mul_mat(const qmm_tensor * src0, const qmm_tensor * src1, const qmm_tensor * dst, qmm_launch_info * out) {
    if (!out) return QMM_ERR_INVALID;
    memset(out, 0, sizeof(*out));
    if (!src0 || !src1 || !dst) return QMM_ERR_INVALID;
    char reason[160];
    WView w;   // shapes only: buffers are not looked at
    if (!mul_mat_ok(src0, src1, dst, false, &w, reason, sizeof(reason))) return QMM_ERR_UNSUPPORTED;
    const int64_t N = src1->ne[1];
    G3Shape g3;
    const bool gemm = use_gemm_for(src0->type, w, N, src1->ne[2] * src1->ne[3]);
    if (gemm && gemm3_shape(src0->type, w, N, src1->ne[2] * src1->ne[3], &g3)) {
        snprintf(out->path, sizeof(out->path), "gemm-stream");
        out->tasks = src1->ne[2] * src1->ne[3];
        out->cols_per_task = 32 * g3.C;
        out->workgroups = g3.workgroups;
        out->threads = g3.threads;
        out->lds_bytes = g3.lds;
        out->k_slices = g3.KS;
        out->k_waves = g3.KS;
        out->tiles_per_wg = g3.U * g3.R / 64;
        out->groups_per_wave = (int32_t)((int64_t)g3.sps * g3.SB / 8);
        return QMM_OK;
    }
    if (gemm) {
        snprintf(out->path, sizeof(out->path), "gemm-mfma");
        out->tasks = src1->ne[2] * src1->ne[3];
        out->cols_per_task = (int32_t)std::min<int64_t>(N, INT32_MAX);
        int threads, lds;
        gemm_shape(src0->type, w, N, out->tasks, &out->workgroups, &threads, &lds);
        out->threads = threads;
        out->lds_bytes = lds;
        out->k_slices = gemm_kslices(src0->type, w, N, out->tasks);
        return QMM_OK;
    }
    FusedPlan fp;
    if (fused_dense_plan(src0->type, w, N, src1->ne[2] * src1->ne[3], &fp, true)) {
        snprintf(out->path, sizeof(out->path), "gemv-fq");
        out->threads = 64 * fp.W;
        out->cols_per_task = fp.nc;
        out->tasks = fp.ntasks;
        out->k_waves = fp.W;
        out->tiles_per_wg = 1;
        out->k_slices = fp.KS;
        out->groups_per_wave = fp.spw;
        out->workgroups = fp.ntasks * w.ntiles * fp.KS;
        out->lds_bytes = fp.lds;
        return QMM_OK;
    }
    const int nc = gemv_task_cols(src0->type, N);
    const int64_t ntasks = (N + nc - 1) / nc * src1->ne[2] * src1->ne[3];
    GemvPlan plan;
    if (!gemv_plan(src0->type, w, nc, ntasks, true, nc >= gemv_mma_min_cols(), &plan)) return QMM_ERR_UNSUPPORTED;
    snprintf(out->path, sizeof(out->path), plan.mma ? "gemv-mfma" : "gemv");
    out->threads = 64 * plan.W;
    out->cols_per_task = nc;
    out->tasks = ntasks;
    out->k_waves = plan.mma ? plan.W / plan.tw : plan.W;
    out->tiles_per_wg = plan.mma ? plan.tw : 1;
    out->k_slices = plan.KS;
    out->groups_per_wave = plan.spw;
    out->workgroups = gemv_workgroups(w, plan);
    out->lds_bytes = (int64_t)gemv_lds_bytes(src0->type, plan);
    return QMM_OK;
}

// a dense fused launch when the shape suits it (false: not taken, nothing enqueued)
static bool try_fused_dense(qmm_ctx * ctx, const qmm_tensor * src0, const qmm_tensor * src1, const WView & w,
                            const GemvDense & dn, float * d, const uint8_t * up_base, int glu, bool noalloc, int * rc) {
    FusedPlan fp;
    if (!fused_dense_plan(src0->type, w, src1->ne[1], dn.ne12 * dn.ne13, &fp, !noalloc)) return false;
    FusedGemv f{};
    if (fp.KS > 1) {
        if ((*rc = ensure_tree(ctx, (size_t)gemv_fused_tree_words(w, fp, glu >= 0)))) return true;
        f.tree = ctx->tree;
    }
    f.x = f32_cols(src1);
    f.K = src1->ne[0];
    f.dense = dn;
    f.base2 = up_base;
    f.glu = glu;
    KTime kt;
    const KTime * ktp = nullptr;
    // (the allocation-free entry point records no timing events)
    if (!noalloc && (*rc = ktime_pair(ctx, &kt, &ktp))) return true;
    const hipError_t e = launch_gemv_fused(src0->type, w, fp, f, d, ctx->sink, ctx->stream, ktp);
    *rc = e == hipSuccess ? ktime_done(ctx) : fail(ctx, QMM_ERR_DEVICE, "launch_gemv_fused: %s", hipGetErrorString(e));
    return true;
}

// MUL_MAT_ID of few tokens with no route: the fused GEMV reads each (slot, token) pair's id
// itself (false: not taken, nothing enqueued)
static bool try_fused_id(qmm_ctx * ctx, const qmm_tensor * src0, const qmm_tensor * src1, const qmm_tensor * ids,
                         const qmm_tensor * dst, const WView & w, const uint8_t * up_base, int glu, int * rc) {
    const int64_t n_used = ids->ne[0], T = ids->ne[1];
    FusedPlan fp;
    if (!fused_id_plan(src0->type, w, n_used, T, &fp)) return false;
    FusedGemv f{};
    f.x = f32_cols(src1);
    f.K = src1->ne[0];
    f.ids = (const char *)ids->buffer->ptr + ids->offs;
    f.ids_nb0 = (int64_t)ids->nb[0];
    f.ids_nb1 = (int64_t)ids->nb[1];
    f.n_used = n_used;
    f.T = T;
    f.ne11 = src1->ne[1];
    f.n_as = src0->ne[2];
    f.dnb1 = (int64_t)(dst->nb[1] / 4);
    f.dnb2 = (int64_t)(dst->nb[2] / 4);
    f.bad_id = ctx->dflags;
    f.base2 = up_base;
    f.glu = glu;
    KTime kt;
    const KTime * ktp = nullptr;
    if ((*rc = ktime_pair(ctx, &kt, &ktp))) return true;
    float * d = (float *)((uint8_t *)dst->buffer->ptr + dst->offs);
    const hipError_t e = launch_gemv_fused(src0->type, w, fp, f, d, ctx->sink, ctx->stream, ktp);
    *rc = e == hipSuccess ? ktime_done(ctx) : fail(ctx, QMM_ERR_DEVICE, "launch_gemv_fused: %s", hipGetErrorString(e));
    return true;
}

// The MUL_MAT after validation: the activation pre-pass, then the GEMV or the GEMM.  With
// `fixed` the activations go to that memory (nothing is allocated, no graph dedup, no kernel
// timing events); otherwise to the context's scratch.
static int mul_mat_launch(qmm_ctx * ctx, const qmm_tensor * src0, const qmm_tensor * src1, const qmm_tensor * dst,
                          const WView & w, const FixedAct * fixed) {
    const int64_t N = src1->ne[1];
    const bool use_gemm = use_gemm_for(src0->type, w, N, src1->ne[2] * src1->ne[3]);
    ActBuf a{};
    int rc;
    float * d = (float *)((uint8_t *)dst->buffer->ptr + dst->offs);
    GemvDense dn;
    dn.ne11 = N;
    dn.ne12 = src1->ne[2];
    dn.ne13 = src1->ne[3];
    dn.r2 = src1->ne[2] / src0->ne[2];
    dn.r3 = src1->ne[3] / src0->ne[3];
    dn.ne02 = src0->ne[2];
    dn.d_nb1 = (int64_t)(dst->nb[1] / 4);
    dn.d_nb2 = (int64_t)(dst->nb[2] / 4);
    dn.d_nb3 = (int64_t)(dst->nb[3] / 4);
    KTime kt;
    const KTime * ktp = nullptr;
    G3Shape g3;
    // weights streamed per wave, dst written once (the shape check is qmm_describe_mul_mat's, so
    // a shape the streaming kernel declines runs on the shared-tile GEMM below, as described)
    if (use_gemm && gemm3_shape(src0->type, w, N, dn.ne12 * dn.ne13, &g3)) {
        const int64_t nbatch = dn.ne12 * dn.ne13;
        TiledAct ta;
        if ((rc = quantize_src1_tiled(ctx, src0->type, src1, w.G, &ta, fixed))) return rc;
        GemmBatch bt;
        bt.ne12 = dn.ne12;
        bt.r2 = dn.r2;
        bt.r3 = dn.r3;
        bt.ne02 = dn.ne02;
        bt.d_nb1 = dn.d_nb1;
        bt.d_nb2 = dn.d_nb2;
        bt.d_nb3 = dn.d_nb3;
        ctx->path = "gemm-stream";
        // the blocks past a whole number per CU in K pieces meeting in tree slots (grown outside
        // captures only; without them, and in qmm_mul_mat_noalloc, the blocks run whole)
        uint32_t * tree = nullptr;
        const size_t tw = gemm3_tree_words(g3);
        if (tw && !fixed) {
            if (!ctx->capturing && (rc = ensure_tree(ctx, tw))) return rc;
            if (ctx->tree_words >= tw) tree = ctx->tree;
        }
        if (!fixed && (rc = ktime_pair(ctx, &kt, &ktp))) return rc;
        QMM_HIP(ctx, launch_gemm3(src0->type, w, ta, nbatch, bt, d, ctx->stream, ktp, tree));
        return ktime_done(ctx);
    }
    if (use_gemm) {
        const int64_t nbatch = dn.ne12 * dn.ne13;
        // K slices add into dst rows from zero_from on (the pre-pass zeroes them)
        const int64_t zero_from = gemm_zero_from(src0->type, w, N, nbatch);
        ZeroJob z{ d, w.M, N * nbatch, N, dn.ne12, dn.d_nb1, dn.d_nb2, dn.d_nb3, zero_from };
        const bool split = zero_from < w.M;
        if ((rc = quantize_src1(ctx, src0->type, src1, true, &a, split ? &z : nullptr, nullptr, fixed))) return rc;
        GemmBatch bt;
        bt.ne12 = dn.ne12;
        bt.r2 = dn.r2;
        bt.r3 = dn.r3;
        bt.ne02 = dn.ne02;
        bt.d_nb1 = dn.d_nb1;
        bt.d_nb2 = dn.d_nb2;
        bt.d_nb3 = dn.d_nb3;
        ctx->path = "gemm-mfma";
        // (every type streams unless the streaming kernels are switched off: QMM_GEMM3=0, or
        // QMM_GEMM3_Q4K / _Q6K / _SBS per type)
        note_downgrade(ctx, "op=MUL_MAT type=%s k=%lld cols=%s path=gemm-mfma reason=no-streaming-gemm",
                       type_name(src0->type), (long long)w.K, cols_bucket(N));
        if (!fixed && (rc = ktime_pair(ctx, &kt, &ktp))) return rc;
        QMM_HIP(ctx, launch_gemm(src0->type, w, a, N, dn.ne12 * dn.ne13, bt, d, ctx->stream, ktp));
        return ktime_done(ctx);
    }
    if (try_fused_dense(ctx, src0, src1, w, dn, d, nullptr, -1, fixed != nullptr, &rc)) {
        ctx->path = "gemv-fq";
        return rc;
    }
    // up to 8 (v_dot4) or 32 (MFMA) columns per task against one weight pass
    const int nc = gemv_task_cols(src0->type, N);
    const int64_t ntasks = (N + nc - 1) / nc * dn.ne12 * dn.ne13;
    GemvPlan plan;
    const bool want_mma = nc >= gemv_mma_min_cols();
    if (!gemv_plan(src0->type, w, nc, ntasks, true, want_mma, &plan))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "mul_mat: GEMV shape out of range");
    ZeroJob z{ d, w.M, N * dn.ne12 * dn.ne13, N, dn.ne12, dn.d_nb1, dn.d_nb2, dn.d_nb3 };
    if ((rc = quantize_src1(ctx, src0->type, src1, false, &a, plan.KS > 1 ? &z : nullptr, nullptr, fixed))) return rc;
    ctx->path = plan.mma ? "gemv-mfma" : "gemv";
    if (N > nc)
        note_downgrade(ctx, "op=MUL_MAT type=%s k=%lld cols=%s path=%s reason=several-weight-passes", type_name(src0->type),
                       (long long)w.K, cols_bucket(N), plan.mma ? "gemv-mfma" : "gemv");
    if (want_mma && !plan.mma)
        note_downgrade(ctx, "op=MUL_MAT type=%s k=%lld cols=%s path=gemv reason=no-mfma-gemv", type_name(src0->type),
                       (long long)w.K, cols_bucket(N));
    if (!fixed && (rc = ktime_pair(ctx, &kt, &ktp))) return rc;
    QMM_HIP(ctx, launch_gemv(src0->type, w, plan, a, nullptr, nullptr, &dn, d, ctx->sink, ctx->stream, ktp));
    return ktime_done(ctx);
}

int qmm_mul_mat(qmm_ctx * ctx, const qmm_tensor * src0, const qmm_tensor * src1, const qmm_tensor * dst) {
    if (!ctx) return QMM_ERR_INVALID;
    char reason[160];
    WView w;
    if (!mul_mat_ok(src0, src1, dst, true, &w, reason, sizeof(reason)))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "mul_mat: %s", reason);
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    return mul_mat_launch(ctx, src0, src1, dst, w, nullptr);
}

int qmm_mul_mat_noalloc(qmm_ctx * ctx, const qmm_tensor * src0, const qmm_tensor * src1, const qmm_tensor * dst) {
    if (!ctx) return QMM_ERR_INVALID;
    char reason[160];
    WView w;
    if (!mul_mat_ok(src0, src1, dst, true, &w, reason, sizeof(reason)))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "mul_mat_noalloc: %s", reason);
    if (!ctx->fixed_scratch) return fail(ctx, QMM_ERR_DEVICE, "mul_mat_noalloc: the device scratch has no address");
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    const FixedAct fixed{ ctx->fixed_scratch, QMM_NOALLOC_SCRATCH_BYTES };
    return mul_mat_launch(ctx, src0, src1, dst, w, &fixed);
}

// The expert tasks of ids into the route scratch (reused inside a graph when ids, ne11, the
// dst strides and the expert count are those of the route already there): pair (i, t) reads
// activation column (i % ne11) + t ne11 and writes dst floats t dnb2 + i dnb1
// with defer, a route that has to run is handed back (*pending) for the quantization launch
// (shared: every token has one more slot, n_used, holding the shared expert: tasks of matrix n_as)
static int route_tasks(qmm_ctx * ctx, const qmm_tensor * ids, int64_t ne11, int64_t n_as, int64_t dnb1, int64_t dnb2,
                       int64_t max_tasks, GemvTask ** tasks, int32_t ** ntasks, PendingRoute * defer = nullptr,
                       bool * pending = nullptr, int shared = 0) {
    if (pending) *pending = false;
    const int64_t n_used = ids->ne[0], T = ids->ne[1], npairs = (n_used + shared) * T;
    const size_t o_tasks = align_up((size_t)npairs * 4, 256);
    const size_t o_cnt = align_up(o_tasks + (size_t)max_tasks * sizeof(GemvTask), 256);
    int rc = ensure(ctx, &ctx->route, &ctx->route_cap, o_cnt + 256);
    if (rc) return rc;
    uint8_t * rb = (uint8_t *)ctx->route;
    *tasks = (GemvTask *)(rb + o_tasks);
    *ntasks = (int32_t *)(rb + o_cnt);
    auto & rk = ctx->rkey;
    const bool hit = ctx->in_graph && rk.valid && rk.gen == ctx->graph_gen && rk.ids.buffer == ids->buffer &&
                     rk.ids.offs == ids->offs && !memcmp(rk.ids.ne, ids->ne, sizeof(ids->ne)) &&
                     !memcmp(rk.ids.nb, ids->nb, sizeof(ids->nb)) && rk.ne11 == ne11 && rk.n_as == n_as &&
                     rk.dnb1 == dnb1 && rk.dnb2 == dnb2 && rk.shared == shared;
    if (hit) return QMM_OK;
    RouteArgs r;
    r.ids = (const int32_t *)((const uint8_t *)ids->buffer->ptr + ids->offs);
    r.ids_nb0 = ids->nb[0];
    r.ids_nb1 = ids->nb[1];
    r.n_used = n_used;
    r.T = T;
    r.ne11 = ne11;
    r.n_as = n_as;
    r.dst_nb1 = dnb1;
    r.dst_nb2 = dnb2;
    r.bad_id = ctx->dflags;
    r.shared = shared;
    if (defer) {
        *defer = PendingRoute{ r, (int32_t *)rb, *tasks, *ntasks };
        *pending = true;
    } else {
        QMM_HIP(ctx, launch_route(r, (int32_t *)rb, *tasks, *ntasks, ctx->stream));
    }
    rk.ids = *ids;
    rk.ne11 = ne11;
    rk.n_as = n_as;
    rk.dnb1 = dnb1;
    rk.dnb2 = dnb2;
    rk.shared = shared;
    rk.gen = ctx->graph_gen;
    rk.valid = ctx->in_graph;
    return QMM_OK;
}

// tasks of one route: (token, slot) pairs of one expert, 1..8 per task, plus the invalid bucket
// (and with the shared expert's slot, its bucket)
static int64_t route_max_tasks(int64_t npairs, int64_t n_as, int shared = 0) {
    return npairs / kMaxTaskCols + std::min(n_as + 1 + shared, npairs) + 1;
}

// The grouped GEMM's route: units of up to 64 pairs of one expert (the invalid ids' bucket
// last), written into the route scratch by the quantization launch (pr).  The GEMV route
// cached there for this graph is gone after this.
static int64_t route_max_units(int64_t npairs, int64_t n_as) {
    return npairs / kUnitCols + std::min(n_as + 1, npairs) + 1;
}
static int route_units(qmm_ctx * ctx, const qmm_tensor * ids, int64_t ne11, int64_t n_as, int64_t dnb1, int64_t dnb2,
                       int64_t max_units, GemmUnit ** units, int32_t ** nunits, PendingRoute * pr) {
    const int64_t n_used = ids->ne[0], T = ids->ne[1], npairs = n_used * T;
    const size_t o_units = align_up((size_t)npairs * 4, 256);
    const size_t o_cnt = align_up(o_units + (size_t)max_units * sizeof(GemmUnit), 256);
    int rc = ensure(ctx, &ctx->route, &ctx->route_cap, o_cnt + 256);
    if (rc) return rc;
    ctx->rkey.valid = false;
    uint8_t * rb = (uint8_t *)ctx->route;
    *units = (GemmUnit *)(rb + o_units);
    *nunits = (int32_t *)(rb + o_cnt);
    RouteArgs r;
    r.ids = (const int32_t *)((const uint8_t *)ids->buffer->ptr + ids->offs);
    r.ids_nb0 = ids->nb[0];
    r.ids_nb1 = ids->nb[1];
    r.n_used = n_used;
    r.T = T;
    r.ne11 = ne11;
    r.n_as = n_as;
    r.dst_nb1 = dnb1;
    r.dst_nb2 = dnb2;
    r.bad_id = ctx->dflags;
    *pr = PendingRoute{ r, (int32_t *)rb, nullptr, *nunits, *units };
    return QMM_OK;
}

// MUL_MAT_ID on the grouped GEMM when the experts average this many pairs or more
// (QMM_MOE_GEMM_MIN overrides; 0 switches it off).  Gate + up + GLU on Q4_K from 64: its GEMV
// tasks fuse both products and the GLU in one launch on the MFMA GEMV, which the grouped GEMM's
// route and two launches overtake only past ~60 pairs (16 experts of 512 x 2048, top-10: 37.3
// against 30.7 us at 40 pairs, 40.2 against 44.1 at 80; IQ4_XS breaks even at 40, Q5_K's v_dot4
// tasks lose from 25)
static int64_t moe_gemm_min_pairs(int type = -1, bool glu = false) {
    const char * e = getenv("QMM_MOE_GEMM_MIN");
    return e ? atoll(e) : glu && type == QMM_TYPE_Q4_K ? 64 : 32;
}
// floats from a MUL_MAT_ID dst's first element to one past its last (the grouped GEMM stores
// through 32-bit byte offsets: it takes spans below 2^30 floats)
static int64_t id_dst_span(const qmm_tensor * dst) {
    return (dst->ne[1] - 1) * (int64_t)(dst->nb[1] / 4) + (dst->ne[2] - 1) * (int64_t)(dst->nb[2] / 4) +
           (dst->ne[3] - 1) * (int64_t)(dst->nb[3] / 4) + dst->ne[0];
}
constexpr int64_t kMaxIdSpan = ((int64_t)1 << 30) - 1;
// the K groups (256 weights) from which the grouped GEMM is taken (QMM_MOE_GEMM_KMIN overrides).
// K = 512, 16 experts of 2048 rows, top-10 at 1024 tokens (640 pairs an expert), grouped
// against the GEMV tasks: Q4_K 121.7 / 130.4 us, Q6_K 130.3 / 185.4, IQ4_XS 130.8 / 166.6; at
// 40 pairs 18.7 / 18.0, 19.4 / 23.5, 19.5 / 21.7.  (Before the gathered stores stopped waiting
// on each offset load, Q4_K lost there: 126 against 110.)  At K = 256 a wave has one stage.
static int64_t moe_gemm_min_groups() {
    const char * e = getenv("QMM_MOE_GEMM_KMIN");
    return e ? atoll(e) : 2;
}
// The grouped GEMM's launch form: 4-wave one-slice blocks, three a CU, when they make a block per
// CU or more and the experts' 64-pair units are mostly full (48 pairs or more on average) or K
// is 512 (split, a wave would have one stage); else the launch rule's shape, which splits K over
// more waves.  Q4_K op, 16 experts of 512 x 2048 top-10 (one-slice against the best split
// shape): 1024 tokens 48.5 against 61.9 us, 512 tokens 35.8 / 38.4, 256 (192 blocks) 27.7 /
// 26.0, 128 (40 pairs a unit) 26.1 / 21.2; 128 experts x 512 tokens top-8 (32 pairs a unit)
// 54.8 / 46.8; 2048 x 512 at 64, 128, 256 and 512 tokens 18.3 / 17.1, 20.7 / 24.1, 26.2 / 32.1
// and 43.5 / 53.4.
static bool moe_one_slice(const WView & w, int64_t npairs, int64_t n_as) {
    const int64_t avg = std::max<int64_t>(1, npairs / n_as), upe = (avg + 63) / 64;
    const int64_t blocks = (2 * w.ntiles + 3) / 4 * n_as * upe;
    return blocks >= 256 && (avg / upe >= 48 || w.G <= 2);
}
static bool use_moe_gemm(int type, const WView & w, int64_t npairs, int64_t n_as, bool glu = false) {
    const int64_t mn = moe_gemm_min_pairs(type, glu);
    G3Shape sh;
    return mn > 0 && npairs >= mn * n_as && w.G >= moe_gemm_min_groups() && gemm3_id_supported(type) &&
           gemm3_id_shape(w, route_max_units(npairs, n_as), moe_one_slice(w, npairs, n_as), &sh);
}

// The route-task path's known costs, as downgrade keys: an expert with more pairs than a task
// takes (8) streams its weights once per task; past the grouped GEMM's pair threshold the type
// has no grouped kernel (Q4_K, Q6_K, Q5_K and IQ4_XS do) or K is below its 512
static void note_moe_downgrades(qmm_ctx * ctx, const char * op, int type, const WView & w, int64_t npairs, int64_t n_as,
                                const char * path, bool glu = false) {
    if (npairs > (int64_t)kMaxTaskCols * n_as)
        note_downgrade(ctx, "op=%s type=%s k=%lld pairs/expert=%s path=%s reason=expert-weights-per-8-pair-task", op,
                       type_name(type), (long long)w.K, cols_bucket((npairs + n_as - 1) / n_as), path);
    const int64_t mn = moe_gemm_min_pairs(type, glu);
    if (mn > 0 && npairs >= mn * n_as)
        note_downgrade(ctx, "op=%s type=%s k=%lld pairs/expert=%s path=%s reason=%s", op, type_name(type),
                       (long long)w.K, cols_bucket((npairs + n_as - 1) / n_as), path,
                       !gemm3_id_supported(type) ? "no-grouped-gemm-for-type" : w.G < moe_gemm_min_groups() ? "grouped-gemm-needs-k-512"
                                                                                    : "grouped-gemm-shape");
}

int qmm_mul_mat_id(qmm_ctx * ctx, const qmm_tensor * src0, const qmm_tensor * src1, const qmm_tensor * ids,
                   const qmm_tensor * dst) {
    if (!ctx) return QMM_ERR_INVALID;
    char reason[160];
    WView w;
    if (!mul_mat_id_ok(src0, src1, ids, dst, true, &w, reason, sizeof(reason)))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "mul_mat_id: %s", reason);
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    const int64_t n_as = src0->ne[2];
    const int64_t npairs = ids->ne[0] * ids->ne[1];
    ActBuf a{};
    int rc;
    if (try_fused_id(ctx, src0, src1, ids, dst, w, nullptr, -1, &rc)) {
        ctx->path = "gemv-id-fq";
        return rc;
    }
    float * dptr = (float *)((uint8_t *)dst->buffer->ptr + dst->offs);
    if (use_moe_gemm(src0->type, w, npairs, n_as) && id_dst_span(dst) <= kMaxIdSpan) {
        const int64_t max_units = route_max_units(npairs, n_as);
        GemmUnit * units;
        int32_t * nunits;
        PendingRoute pr;
        if ((rc = route_units(ctx, ids, src1->ne[1], n_as, (int64_t)(dst->nb[1] / 4), (int64_t)(dst->nb[2] / 4),
                              max_units, &units, &nunits, &pr)))
            return rc;
        if ((rc = quantize_src1(ctx, src0->type, src1, false, &a, nullptr, &pr))) return rc;
        ctx->path = "gemm-id-stream";
        KTime kt;
        const KTime * ktp;
        if ((rc = ktime_pair(ctx, &kt, &ktp))) return rc;
        QMM_HIP(ctx, launch_gemm3_id(src0->type, w, a, units, nunits, max_units, moe_one_slice(w, npairs, n_as), dptr,
                                     id_dst_span(dst), ctx->stream, ktp));
        return ktime_done(ctx);
    }
    const int64_t max_tasks = route_max_tasks(npairs, n_as);
    const int nc = (int)std::min<int64_t>(kMaxTaskCols, npairs);
    GemvPlan plan;
    // tasks carry 1..8 pairs each: the MFMA kernel pays off when experts average two or more
    if (!gemv_plan(src0->type, w, nc, max_tasks, false, npairs >= 2 * n_as, &plan))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "mul_mat_id: GEMV shape out of range");
    GemvTask * tasks;
    int32_t * ntasks;
    PendingRoute pr;
    bool pending;
    if ((rc = route_tasks(ctx, ids, src1->ne[1], n_as, (int64_t)(dst->nb[1] / 4), (int64_t)(dst->nb[2] / 4), max_tasks,
                          &tasks, &ntasks, &pr, &pending)))
        return rc;
    if ((rc = quantize_src1(ctx, src0->type, src1, false, &a, nullptr, pending ? &pr : nullptr))) {
        ctx->rkey.valid = false;                                  // the route may not have run
        return rc;
    }
    float * d = (float *)((uint8_t *)dst->buffer->ptr + dst->offs);
    ctx->path = plan.mma ? "gemv-id-mfma" : "gemv-id";
    note_moe_downgrades(ctx, "MUL_MAT_ID", src0->type, w, npairs, n_as, ctx->path.c_str());
    KTime kt;
    const KTime * ktp;
    if ((rc = ktime_pair(ctx, &kt, &ktp))) return rc;
    QMM_HIP(ctx, launch_gemv(src0->type, w, plan, a, tasks, ntasks, nullptr, d, ctx->sink, ctx->stream, ktp));
    return ktime_done(ctx);
}

// MUL_MAT_ID (gate experts), MUL_MAT_ID (up experts) and the GLU, the MoE form of
// qmm_mul_mat_glu (the reference's MUL_MAT_ID + GLU fuse; its audit,
// docs/campaigns/research-concept-mining/ipex-llm/audit.md:83-87): one activation
// quantization, one route, one GEMV launch over both stacks.  With enough tasks to fill the
// chip, each work-group streams its tile of the gate stack, then of the up stack, against the
// same activations and stores act(gate) * up (task lists never split K over work-groups, so
// each holds whole sums): no scratch and no GLU launch.  With few (decode), the list runs once
// on each stack in parallel into a scratch [2][T][n_used][M] and the GLU kernel writes dst:
// twice the work-groups for a latency-bound launch (config 3 at T = 1: 17.2 against 22.4 us
// per call, at T = 256 127 against 123).
int qmm_mul_mat_id_glu(qmm_ctx * ctx, const qmm_tensor * gate, const qmm_tensor * up, const qmm_tensor * src1,
                       const qmm_tensor * ids, const qmm_tensor * dst, int32_t glu_op) {
    if (!ctx) return QMM_ERR_INVALID;
    if (glu_op != QMM_GLU_REGLU && glu_op != QMM_GLU_GEGLU && glu_op != QMM_GLU_SWIGLU && glu_op != QMM_GLU_GEGLU_ERF &&
        glu_op != QMM_GLU_GEGLU_QUICK)
        return fail(ctx, QMM_ERR_UNSUPPORTED, "mul_mat_id_glu: GLU op %d", glu_op);
    char reason[160];
    WView wg, wu;
    if (!mul_mat_id_ok(gate, src1, ids, dst, true, &wg, reason, sizeof(reason)))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "mul_mat_id_glu: gate: %s", reason);
    if (!mul_mat_id_ok(up, src1, ids, dst, true, &wu, reason, sizeof(reason)))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "mul_mat_id_glu: up: %s", reason);
    if (up->type != gate->type || memcmp(gate->ne, up->ne, sizeof(gate->ne)))
        return fail(ctx, QMM_ERR_INVALID, "mul_mat_id_glu: gate and up must be one type and shape");
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    const int64_t M = gate->ne[1], n_as = gate->ne[2], n_used = ids->ne[0], T = ids->ne[1], npairs = n_used * T;
    ActBuf a{};
    int rc;
    if (try_fused_id(ctx, gate, src1, ids, dst, wg, wu.base, glu_op, &rc)) {
        ctx->path = "glu-gemv-id-fq";
        return rc;
    }
    if (use_moe_gemm(gate->type, wg, npairs, n_as, true) && id_dst_span(dst) <= kMaxIdSpan) {
        // the grouped GEMM: one route and quantization for both products; gate into the scratch
        // at dst's offsets, then up with act(gate) * up applied at its stores
        const int64_t dnb1 = (int64_t)(dst->nb[1] / 4), dnb2 = (int64_t)(dst->nb[2] / 4);
        const int64_t span = id_dst_span(dst);
        if ((rc = ensure(ctx, &ctx->glu, &ctx->glu_cap, (size_t)span * sizeof(float)))) return rc;
        const int64_t max_units = route_max_units(npairs, n_as);
        GemmUnit * units;
        int32_t * nunits;
        PendingRoute pr;
        if ((rc = route_units(ctx, ids, src1->ne[1], n_as, dnb1, dnb2, max_units, &units, &nunits, &pr))) return rc;
        if ((rc = quantize_src1(ctx, gate->type, src1, false, &a, nullptr, &pr))) return rc;
        float * g = (float *)ctx->glu;
        float * d = (float *)((uint8_t *)dst->buffer->ptr + dst->offs);
        const bool one = moe_one_slice(wg, npairs, n_as);
        QMM_HIP(ctx, launch_gemm3_id(gate->type, wg, a, units, nunits, max_units, one, g, span, ctx->stream));
        QMM_HIP(ctx, launch_gemm3_id(up->type, wu, a, units, nunits, max_units, one, d, span, ctx->stream, nullptr, g,
                                     glu_op));
        ctx->path = "glu-gemm-id-stream";
        return QMM_OK;
    }
    const int64_t max_tasks = route_max_tasks(npairs, n_as);
    const int nc = (int)std::min<int64_t>(kMaxTaskCols, npairs);
    const bool in_wg = max_tasks * wg.ntiles >= 1024;             // enough work-groups to fill the chip
    GemvPlan plan;
    if (!gemv_plan(gate->type, wg, nc, in_wg ? max_tasks : 2 * max_tasks, false, npairs >= 2 * n_as, &plan))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "mul_mat_id_glu: GEMV shape out of range");
    const size_t half = (size_t)(M * npairs);
    float * sg = nullptr;
    if (!in_wg) {
        if ((rc = ensure(ctx, &ctx->glu, &ctx->glu_cap, 2 * half * sizeof(float)))) return rc;
        sg = (float *)ctx->glu;
    }
    GemvTask * tasks;
    int32_t * ntasks;
    // in_wg: the dst's strides; else the scratch halves, contiguous [T][n_used][M]
    const int64_t dnb1 = in_wg ? (int64_t)(dst->nb[1] / 4) : M, dnb2 = in_wg ? (int64_t)(dst->nb[2] / 4) : M * n_used;
    PendingRoute pr;
    bool pending;
    if ((rc = route_tasks(ctx, ids, src1->ne[1], n_as, dnb1, dnb2, max_tasks, &tasks, &ntasks, &pr, &pending))) return rc;
    if ((rc = quantize_src1(ctx, gate->type, src1, false, &a, nullptr, pending ? &pr : nullptr))) {
        ctx->rkey.valid = false;                                  // the route may not have run
        return rc;
    }
    GemvPair pair{ wu.base, in_wg ? 0 : (int64_t)half, in_wg ? glu_op : -1 };
    float * d = (float *)((uint8_t *)dst->buffer->ptr + dst->offs);
    ctx->path = plan.mma ? "glu-gemv-id-mfma" : "glu-gemv-id";
    note_moe_downgrades(ctx, "MUL_MAT_ID+GLU", gate->type, wg, npairs, n_as, ctx->path.c_str(), true);
    KTime kt;
    const KTime * ktp;
    if ((rc = ktime_pair(ctx, &kt, &ktp))) return rc;
    QMM_HIP(ctx, launch_gemv(gate->type, wg, plan, a, tasks, ntasks, nullptr, in_wg ? d : sg, ctx->sink, ctx->stream, ktp,
                             &pair));
    if ((rc = ktime_done(ctx))) return rc;
    if (in_wg) return QMM_OK;
    GluArgs g;
    g.gate = sg;
    g.up = sg + half;
    g.dst = d;
    g.M = M;
    g.N = n_used;
    g.nb = T;
    g.ne12 = T;
    g.d_nb1 = (int64_t)(dst->nb[1] / 4);
    g.d_nb2 = (int64_t)(dst->nb[2] / 4);
    g.d_nb3 = 0;
    QMM_HIP(ctx, launch_glu(glu_op, g, ctx->stream));
    return QMM_OK;
}

int qmm_moe_topk(qmm_ctx * ctx, const qmm_tensor * logits, const qmm_tensor * ids, const qmm_tensor * weights,
                 float cmin, float cmax) {
    if (!ctx) return QMM_ERR_INVALID;
    if (!check_f32(logits) || !check_f32(weights) || !ids || !ids->buffer || ids->type != QMM_TYPE_I32 || ids->nb[0] != 4)
        return fail(ctx, QMM_ERR_INVALID, "moe_topk: logits / weights f32 and ids i32 with nb[0] == 4");
    const int64_t n_expert = logits->ne[0], T = logits->ne[1], k = ids->ne[0];
    if (logits->ne[2] != 1 || logits->ne[3] != 1 || ids->ne[1] != T || ids->ne[2] != 1 || ids->ne[3] != 1 ||
        weights->ne[0] != k || weights->ne[1] != T || weights->ne[2] != 1 || weights->ne[3] != 1)
        return fail(ctx, QMM_ERR_INVALID, "moe_topk: logits [n_expert, T], ids and weights [k, T]");
    if (n_expert > 1024 || k < 1 || k > 32 || k > n_expert)
        return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_topk: n_expert <= 1024 and 1 <= k <= min(32, n_expert)");
    if (!span_ok(logits) || !span_ok(ids) || !span_ok(weights) || logits->nb[1] % 4 || ids->nb[1] % 4 ||
        weights->nb[1] % 4 || logits->offs % 4 || ids->offs % 4 || weights->offs % 4)
        return fail(ctx, QMM_ERR_INVALID, "moe_topk: a view past its buffer or not 4-byte aligned");
    if (!(cmin <= cmax) || !(cmax > 0.0f)) return fail(ctx, QMM_ERR_INVALID, "moe_topk: clamp range");
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    TopkArgs a;
    a.logits = (const char *)logits->buffer->ptr + logits->offs;
    a.ids = (char *)ids->buffer->ptr + ids->offs;
    a.w = (char *)weights->buffer->ptr + weights->offs;
    a.nbl1 = (int64_t)logits->nb[1];
    a.nbi1 = (int64_t)ids->nb[1];
    a.nbw1 = (int64_t)weights->nb[1];
    a.n_expert = (int)n_expert;
    a.k = (int)k;
    a.n_tok = T;
    a.cmin = cmin;
    a.cmax = cmax;
    ctx->path = "moe-topk";
    QMM_HIP(ctx, launch_topk(a, ctx->stream));
    return QMM_OK;
}

int qmm_moe_combine(qmm_ctx * ctx, const qmm_tensor * experts, const qmm_tensor * weights, const qmm_tensor * shared,
                    const qmm_tensor * gate, const qmm_tensor * dst) {
    if (!ctx) return QMM_ERR_INVALID;
    if (!check_f32(experts) || !check_f32(weights) || !check_f32(dst) || (shared && !check_f32(shared)) ||
        (gate && !check_f32(gate)) || (!shared) != (!gate))
        return fail(ctx, QMM_ERR_INVALID, "moe_combine: f32 tensors with nb[0] == 4; shared and gate together");
    const int64_t M = experts->ne[0], k = experts->ne[1], T = experts->ne[2];
    if (experts->ne[3] != 1 || weights->ne[0] != k || weights->ne[1] != T || weights->ne[2] != 1 || dst->ne[0] != M ||
        dst->ne[1] != T || dst->ne[2] != 1 || (shared && (shared->ne[0] != M || shared->ne[1] != T || shared->ne[2] != 1)) ||
        (gate && (gate->ne[0] != 1 || gate->ne[1] != T || gate->ne[2] != 1)))
        return fail(ctx, QMM_ERR_INVALID, "moe_combine: experts [M, k, T], weights [k, T], shared and dst [M, T], gate [1, T]");
    if (k < 1 || k > 64) return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_combine: 1 <= k <= 64");
    for (const qmm_tensor * t : { experts, weights, dst, shared, gate }) {
        if (t && (!span_ok(t) || t->offs % 4 || t->nb[1] % 4 || t->nb[2] % 4))
            return fail(ctx, QMM_ERR_INVALID, "moe_combine: a view past its buffer or not 4-byte aligned");
    }
    if (ranges_overlap(dst, experts) || ranges_overlap(dst, weights) || ranges_overlap(dst, shared) || ranges_overlap(dst, gate))
        return fail(ctx, QMM_ERR_INVALID, "moe_combine: dst overlaps an input");
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    CombineArgs a{};
    a.experts = (const char *)experts->buffer->ptr + experts->offs;
    a.w = (const char *)weights->buffer->ptr + weights->offs;
    a.shared = shared ? (const char *)shared->buffer->ptr + shared->offs : nullptr;
    a.gate = gate ? (const char *)gate->buffer->ptr + gate->offs : nullptr;
    a.dst = (char *)dst->buffer->ptr + dst->offs;
    a.M = M;
    a.T = T;
    a.k = (int)k;
    a.enb1 = (int64_t)experts->nb[1];
    a.enb2 = (int64_t)experts->nb[2];
    a.wnb1 = (int64_t)weights->nb[1];
    a.snb1 = shared ? (int64_t)shared->nb[1] : 0;
    a.gnb1 = gate ? (int64_t)gate->nb[1] : 0;
    a.dnb1 = (int64_t)dst->nb[1];
    ctx->path = "moe-combine";
    QMM_HIP(ctx, launch_combine(a, ctx->stream));
    return QMM_OK;
}

// A MoE FFN block in two launches of the fused GEMV (decode token counts):
//  1. every (slot, token) pair's gate and up rows and their GLU, the shared expert as one more
//     slot of every token, into a context scratch h [T][slots][M] (with the router's logits:
//     every work-group first ranks its token, and tile 0 of slot 0 stores the ids and weights);
//  2. every pair's down rows from its h column, times its router weight (the shared slot's by
//     the sigmoid of its gate logit), the token's slots added in the exchange tree, the root
//     storing dst's row.
// Replaces MUL_MAT_ID gate, MUL_MAT_ID up, GLU, MUL_MAT_ID down, MUL by the weights, the ADDs
// over the slots and the shared expert's MUL_MATs, GLU, sigmoid and ADD: five dependent launches
// of the op-by-op chain, six with the router.  The slot sums are taken in the tree's pairwise
// order instead of slot by slot.
static bool glu_op_ok(int32_t op) {
    return op == QMM_GLU_REGLU || op == QMM_GLU_GEGLU || op == QMM_GLU_SWIGLU || op == QMM_GLU_GEGLU_ERF ||
           op == QMM_GLU_GEGLU_QUICK;
}

// The MoE FFN block at 16 tokens or more: the router (when given logits), then one route and
// activation quantization, the gate/up + GLU products over the route's tasks, the down
// product's route and quantization, its products, and the combine - with the shared expert as
// one more slot of every token in both routes (bucket n_as: tasks of matrix n_as read its
// images), so it streams inside the routed launches on their quantization instead of running
// as its own five launches.  h [M][slots][T] and the expert rows [OUT][slots][T] live in the
// context's scratch.
static int moe_ffn_route(qmm_ctx * ctx, const qmm_moe_ffn_args * args, int type, const WView & wg, const WView & wu,
                         const WView & wd, const WView & wsg, const WView & wsu, const WView & wsd, int64_t HID, int64_t M,
                         int64_t OUT, int64_t n_as, int64_t n_used, int64_t T, bool sh, bool xt2, bool dt2) {
    const qmm_tensor *x = args->x, *ids = args->ids, *weights = args->weights, *dst = args->dst;
    const int shared = sh ? 1 : 0;
    const int64_t nsl = n_used + shared, npairs = nsl * T;
    int rc;
    // experts averaging the grouped GEMM's pair count stream faster through the ops' grouped
    // GEMM than through 8-column tasks: decline, nothing enqueued
    if (use_moe_gemm(type, wg, n_used * T, n_as) || use_moe_gemm(type, wd, n_used * T, n_as))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_ffn: the experts' pairs take the grouped GEMM: run the ops");
    const int64_t max_tasks = route_max_tasks(npairs, n_as, shared);
    const int nc = (int)std::min<int64_t>(kMaxTaskCols, npairs);
    const bool in_wg = max_tasks * wg.ntiles >= 1024;             // as qmm_mul_mat_id_glu
    GemvPlan p1, p2;
    if (!gemv_plan(type, wg, nc, in_wg ? max_tasks : 2 * max_tasks, false, npairs >= 2 * n_as, &p1) ||
        !gemv_plan(type, wd, nc, max_tasks, false, npairs >= 2 * n_as, &p2))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_ffn: GEMV shape out of range");
    if (args->logits) {
        if ((rc = qmm_moe_topk(ctx, args->logits, ids, weights, args->cmin, args->cmax))) return rc;
    }
    // scratch: h, then the expert rows, then (the few-work-group form) the gate and up halves
    const size_t hb = (size_t)(M * npairs), eb = (size_t)(OUT * npairs);
    if ((rc = ensure(ctx, &ctx->glu, &ctx->glu_cap, (hb + eb + (in_wg ? 0 : 2 * hb)) * sizeof(float)))) return rc;
    float * h = (float *)ctx->glu, * ex = h + hb, * sg = ex + eb;
    qmm_buffer scratch{ ctx->glu, ctx->glu_cap };
    // x as MUL_MAT_ID's src1 [HID, 1, T]
    qmm_tensor xs = *x;
    xs.ne[0] = HID;
    xs.ne[1] = 1;
    xs.ne[2] = T;
    xs.ne[3] = 1;
    xs.nb[2] = xt2 ? x->nb[1] : x->nb[2];
    xs.nb[3] = xs.nb[2] * (size_t)T;
    // gate/up + GLU into h
    GemvTask * tasks;
    int32_t * ntasks;
    PendingRoute pr;
    bool pending;
    ActBuf a{};
    if ((rc = route_tasks(ctx, ids, 1, n_as, M, M * nsl, max_tasks, &tasks, &ntasks, &pr, &pending, shared))) return rc;
    if ((rc = quantize_src1(ctx, type, &xs, false, &a, nullptr, pending ? &pr : nullptr))) {
        ctx->rkey.valid = false;
        return rc;
    }
    GemvPair gp;
    gp.base2 = wu.base;
    gp.up_doff = in_wg ? 0 : (int64_t)hb;
    gp.glu = in_wg ? args->glu_op : -1;
    gp.sh_mat = sh ? (int32_t)n_as : -1;
    gp.sh_base = wsg.base;
    gp.sh_base2 = wsu.base;
    QMM_HIP(ctx, launch_gemv(type, wg, p1, a, tasks, ntasks, nullptr, in_wg ? h : sg, ctx->sink, ctx->stream, nullptr, &gp));
    if (!in_wg) {
        GluArgs g;
        g.gate = sg;
        g.up = sg + hb;
        g.dst = h;
        g.M = M;
        g.N = nsl;
        g.nb = T;
        g.ne12 = T;
        g.d_nb1 = M;
        g.d_nb2 = M * nsl;
        g.d_nb3 = 0;
        QMM_HIP(ctx, launch_glu(args->glu_op, g, ctx->stream));
    }
    // down over h [M, slots, T] into the expert rows [OUT, slots, T]
    qmm_tensor hs{};
    hs.type = QMM_TYPE_F32;
    hs.buffer = &scratch;
    hs.offs = 0;
    hs.ne[0] = M;
    hs.ne[1] = nsl;
    hs.ne[2] = T;
    hs.ne[3] = 1;
    hs.nb[0] = 4;
    hs.nb[1] = (size_t)M * 4;
    hs.nb[2] = (size_t)(M * nsl) * 4;
    hs.nb[3] = hs.nb[2] * (size_t)T;
    ActBuf a2{};
    if ((rc = route_tasks(ctx, ids, nsl, n_as, OUT, OUT * nsl, max_tasks, &tasks, &ntasks, &pr, &pending, shared))) return rc;
    rc = quantize_src1(ctx, type, &hs, false, &a2, nullptr, pending ? &pr : nullptr);
    ctx->key.valid = false;                                       // (h's buffer is this call's own)
    ctx->rkey.valid = false;
    if (rc) return rc;
    GemvPair dp;
    dp.base2 = nullptr;
    dp.up_doff = 0;
    dp.glu = -1;
    dp.sh_mat = sh ? (int32_t)n_as : -1;
    dp.sh_base = wsd.base;
    QMM_HIP(ctx, launch_gemv(type, wd, p2, a2, tasks, ntasks, nullptr, ex, ctx->sink, ctx->stream, nullptr, &dp));
    // the routed rows times their weights in slot order, then the (gated) shared row
    CombineArgs c{};
    c.experts = (const char *)ex;
    c.w = (const char *)weights->buffer->ptr + weights->offs;
    c.shared = sh ? (const char *)(ex + n_used * OUT) : nullptr;
    c.gate = args->shared_logit ? (const char *)args->shared_logit->buffer->ptr + args->shared_logit->offs : nullptr;
    c.dst = (char *)dst->buffer->ptr + dst->offs;
    c.M = OUT;
    c.T = T;
    c.k = (int)n_used;
    c.enb1 = OUT * 4;
    c.enb2 = OUT * nsl * 4;
    c.wnb1 = (int64_t)weights->nb[1];
    c.snb1 = OUT * nsl * 4;
    c.gnb1 = args->shared_logit ? (int64_t)args->shared_logit->nb[1] : 0;
    c.dnb1 = (int64_t)(dt2 ? dst->nb[1] : dst->nb[2]);
    QMM_HIP(ctx, launch_combine(c, ctx->stream));
    ctx->path = "moe-ffn-route";
    return QMM_OK;
}

int qmm_moe_ffn(qmm_ctx * ctx, const qmm_moe_ffn_args * args) {
    if (!ctx) return QMM_ERR_INVALID;
    if (!args) return fail(ctx, QMM_ERR_INVALID, "moe_ffn: null args");
    const qmm_tensor *gate = args->gate_exps, *up = args->up_exps, *down = args->down_exps, *x = args->x;
    const qmm_tensor *ids = args->ids, *weights = args->weights, *dst = args->dst, *logits = args->logits;
    const qmm_tensor *sgate = args->shared_gate, *sup = args->shared_up, *sdown = args->shared_down;
    const qmm_tensor * slogit = args->shared_logit;
    const int32_t glu_op = args->glu_op;
    if (!glu_op_ok(glu_op)) return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_ffn: GLU op %d", glu_op);
    if (!gate || !up || !down || !x || !ids || !weights || !dst) return fail(ctx, QMM_ERR_INVALID, "moe_ffn: null tensor");
    const bool sh = sgate || sup || sdown;
    if (sh && !(sgate && sup && sdown))
        return fail(ctx, QMM_ERR_INVALID, "moe_ffn: the shared expert's gate, up and down: all or none");
    if (slogit && !sh) return fail(ctx, QMM_ERR_INVALID, "moe_ffn: a shared gate logit without a shared expert");
    char reason[160];
    WView wg, wu, wd, wsg{}, wsu{}, wsd{};
    if (!weight_image(gate, true, &wg, reason, sizeof(reason)) || !weight_image(up, true, &wu, reason, sizeof(reason)) ||
        !weight_image(down, true, &wd, reason, sizeof(reason)))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_ffn: experts: %s", reason);
    const int type = gate->type;
    if (up->type != type || down->type != type || memcmp(gate->ne, up->ne, sizeof(gate->ne)) || gate->ne[3] != 1 ||
        down->ne[3] != 1)
        return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_ffn: gate, up and down experts of one type, gate and up of one shape");
    const int64_t HID = gate->ne[0], M = gate->ne[1], n_as = gate->ne[2], OUT = down->ne[1];
    if (down->ne[0] != M || down->ne[2] != n_as)
        return fail(ctx, QMM_ERR_INVALID, "moe_ffn: down experts must be [M, n_out, n_as] with gate's M and n_as");
    if (n_as > 8192) return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_ffn: more than 8192 experts");
    if ((HID % 256 || M % 256) && vec_dot_type(type) == QMM_TYPE_Q8_K)
        return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_ffn: K is not a multiple of 256");
    if (sh) {
        if (!weight_image(sgate, true, &wsg, reason, sizeof(reason)) || !weight_image(sup, true, &wsu, reason, sizeof(reason)) ||
            !weight_image(sdown, true, &wsd, reason, sizeof(reason)))
            return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_ffn: shared expert: %s", reason);
        if (sgate->type != type || sup->type != type || sdown->type != type || sgate->ne[0] != HID ||
            sgate->ne[1] != M || sgate->ne[2] != 1 || sgate->ne[3] != 1 || memcmp(sgate->ne, sup->ne, sizeof(sgate->ne)) ||
            sdown->ne[0] != M || sdown->ne[1] != OUT || sdown->ne[2] != 1 || sdown->ne[3] != 1)
            return fail(ctx, QMM_ERR_UNSUPPORTED,
                        "moe_ffn: the shared expert must have the routed experts' type and matrix shapes (run the ops "
                        "one by one)");
    }
    const int64_t n_used = ids->ne[0], T = ids->ne[1];
    if (ids->type != QMM_TYPE_I32 || ids->nb[0] != 4 || !ids->buffer || ids->ne[2] != 1 || ids->ne[3] != 1 ||
        !span_ok(ids) || ids->nb[1] % 4 || ids->offs % 4)
        return fail(ctx, QMM_ERR_INVALID, "moe_ffn: ids must be i32 [n_used, T] with nb[0] == 4");
    if (!check_f32(weights) || weights->ne[0] != n_used || weights->ne[1] != T || weights->ne[2] != 1 ||
        weights->ne[3] != 1 || !span_ok(weights) || weights->nb[1] % 4 || weights->offs % 4)
        return fail(ctx, QMM_ERR_INVALID, "moe_ffn: weights must be f32 [n_used, T]");
    // x: [HID, T] or [HID, 1, T]; dst: [n_out, T] or [n_out, 1, T] (token t's row at t dnb floats)
    const bool xt2 = x->ne[1] == T && x->ne[2] == 1, dt2 = dst->ne[1] == T && dst->ne[2] == 1;
    if (!check_f32(x) || x->ne[0] != HID || !(xt2 || (x->ne[1] == 1 && x->ne[2] == T)) || x->ne[3] != 1 ||
        !span_ok(x) || x->nb[1] % 4 || x->nb[2] % 4 || x->offs % 4)
        return fail(ctx, QMM_ERR_INVALID, "moe_ffn: x must be f32 [K, T] or [K, 1, T] with K the experts' ne0");
    if (!check_f32(dst) || dst->ne[0] != OUT || !(dt2 || (dst->ne[1] == 1 && dst->ne[2] == T)) || dst->ne[3] != 1 ||
        !span_ok(dst) || dst->nb[1] % 4 || dst->nb[2] % 4 || dst->offs % 4)
        return fail(ctx, QMM_ERR_INVALID, "moe_ffn: dst must be f32 [n_out, T] or [n_out, 1, T]");
    if (slogit && (!check_f32(slogit) || slogit->ne[0] != 1 || slogit->ne[1] != T || slogit->ne[2] != 1 ||
                   slogit->ne[3] != 1 || !span_ok(slogit) || slogit->nb[1] % 4 || slogit->offs % 4))
        return fail(ctx, QMM_ERR_INVALID, "moe_ffn: the shared gate logit must be f32 [1, T]");
    if (logits) {
        if (!check_f32(logits) || logits->ne[0] != n_as || logits->ne[1] != T || logits->ne[2] != 1 ||
            logits->ne[3] != 1 || !span_ok(logits) || logits->nb[1] % 4 || logits->offs % 4)
            return fail(ctx, QMM_ERR_INVALID, "moe_ffn: router logits must be f32 [n_as, T]");
        if (n_as > 1024 || n_used < 1 || n_used > 32 || n_used > n_as)
            return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_ffn: the router takes n_as <= 1024 and 1 <= n_used <= min(32, n_as)");
    }
    const int64_t nsl = n_used + (sh ? 1 : 0);
    if (n_used > 64) return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_ffn: more than 64 slots a token");
    if (!fused_on() || T >= moe_direct_tokens()) {
        QMM_HIP(ctx, hipSetDevice(ctx->device));
        return moe_ffn_route(ctx, args, type, wg, wu, wd, wsg, wsu, wsd, HID, M, OUT, n_as, n_used, T, sh, xt2, dt2);
    }
    FusedPlan p1, p2;
    if (!gemv_fused_plan(type, wg, 1, nsl * T, gemv_fused_waves_target(), &p1) ||
        !gemv_fused_plan(type, wd, 1, nsl * T, gemv_fused_waves_target(), &p2) || nsl > 65535 ||
        nsl * T * wd.ntiles >= 0x7fffffff)
        return fail(ctx, QMM_ERR_UNSUPPORTED, "moe_ffn: fused GEMV shape out of range");
    // the down launch: once its (tile, token) work-groups fill the CUs, a work-group per (tile,
    // token) whose waves are the token's slots, each over the whole K, their rows added in slot
    // order through LDS (the graph's ADD order, no tree); fewer tokens: one work-group per (tile,
    // slot, token), spreading the slots over more CUs, the slots meeting in the tree (config 3
    // layer: T = 1 17.6 against 20.0 us, T = 4 even, T = 8 35.2 against 33.4-34.3, T = 15 58.5
    // against 56.4).  QMM_MOE_SLOTW: 0 the tree, 1 the slot waves when they fit (tests).
    const char * sw = getenv("QMM_MOE_SLOTW");
    const bool slotw = (sw ? atoi(sw) != 0 : T * wd.ntiles >= 256) && gemv_fused_slot_plan(type, wd, nsl, T, &p2);
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    int rc;
    const size_t hbytes = (size_t)(M * nsl * T) * sizeof(float);
    if ((rc = ensure(ctx, &ctx->glu, &ctx->glu_cap, hbytes))) return rc;
    if (!slotw && (rc = ensure_tree(ctx, (size_t)(T * wd.ntiles * 2 * nsl * 64)))) return rc;
    float * h = (float *)ctx->glu;
    const char * idp = (const char *)ids->buffer->ptr + ids->offs;

    FusedGemv f1{};
    f1.x = f32_cols(x);
    f1.K = HID;
    f1.ids = idp;
    f1.ids_nb0 = 4;
    f1.ids_nb1 = (int64_t)ids->nb[1];
    f1.n_used = n_used;
    f1.T = T;
    f1.ne11 = 1;
    f1.n_as = n_as;
    f1.dnb1 = M;
    f1.dnb2 = M * nsl;
    f1.bad_id = ctx->dflags;
    f1.base2 = wu.base;
    f1.glu = glu_op;
    f1.n_shared = sh ? 1 : 0;
    f1.sh_base = wsg.base;
    f1.sh_base2 = wsu.base;
    if (logits) {
        f1.lg = (const float *)((const char *)logits->buffer->ptr + logits->offs);
        f1.lg_nb1 = (int64_t)(logits->nb[1] / 4);
        f1.n_expert = (int)n_as;
        f1.cmin = args->cmin;
        f1.cmax = args->cmax;
        f1.wout = (float *)((char *)weights->buffer->ptr + weights->offs);
        f1.wout_nb1 = (int64_t)(weights->nb[1] / 4);
    }
    hipError_t e = launch_gemv_fused(type, wg, p1, f1, h, ctx->sink, ctx->stream, nullptr);
    if (e != hipSuccess) return fail(ctx, QMM_ERR_DEVICE, "moe_ffn: gate/up launch: %s", hipGetErrorString(e));

    FusedGemv f2{};
    f2.x.base = (const char *)h;                                  // h column i + t nsl
    f2.x.ne1 = nsl * T;
    f2.x.ne2 = 1;
    f2.x.nb1 = (size_t)M * sizeof(float);
    f2.x.nb2 = f2.x.nb3 = (size_t)(M * nsl * T) * sizeof(float);
    f2.K = M;
    f2.ids = idp;
    f2.ids_nb0 = 4;
    f2.ids_nb1 = (int64_t)ids->nb[1];
    f2.n_used = n_used;
    f2.T = T;
    f2.ne11 = nsl;
    f2.n_as = n_as;
    f2.bad_id = ctx->dflags;
    f2.glu = -1;
    f2.tree = ctx->tree;
    f2.n_shared = sh ? 1 : 0;
    f2.sh_base = wsd.base;
    f2.comb = slotw ? 2 : 1;
    f2.cw = (const float *)((const char *)weights->buffer->ptr + weights->offs);
    f2.cw_nb0 = 1;
    f2.cw_nb1 = (int64_t)(weights->nb[1] / 4);
    f2.sl = slogit ? (const float *)((const char *)slogit->buffer->ptr + slogit->offs) : nullptr;
    f2.sl_nb1 = slogit ? (int64_t)(slogit->nb[1] / 4) : 0;
    f2.d_nb1 = (int64_t)((dt2 ? dst->nb[1] : dst->nb[2]) / 4);
    float * d = (float *)((uint8_t *)dst->buffer->ptr + dst->offs);
    e = launch_gemv_fused(type, wd, p2, f2, d, ctx->sink, ctx->stream, nullptr);
    if (e != hipSuccess) return fail(ctx, QMM_ERR_DEVICE, "moe_ffn: down/combine launch: %s", hipGetErrorString(e));
    ctx->path = "moe-ffn-fq";
    return QMM_OK;
}

// MUL_MAT, MUL_MAT, GLU of an FFN (the chain the reference's fuse_mm_glu takes): the gate and up
// sums go to a context scratch [2][batch][N][M], then the GLU kernel writes dst.  At GEMV widths
// with one batch and one weight type a single GEMV launch streams both images (matrix 1 of the
// launch is up's image, both read the same activation columns); otherwise two MUL_MATs share one
// activation quantization.
int qmm_mul_mat_glu(qmm_ctx * ctx, const qmm_tensor * gate, const qmm_tensor * up, const qmm_tensor * src1,
                    const qmm_tensor * dst, int32_t glu_op) {
    if (!ctx) return QMM_ERR_INVALID;
    if (glu_op != QMM_GLU_REGLU && glu_op != QMM_GLU_GEGLU && glu_op != QMM_GLU_SWIGLU && glu_op != QMM_GLU_GEGLU_ERF &&
        glu_op != QMM_GLU_GEGLU_QUICK)
        return fail(ctx, QMM_ERR_UNSUPPORTED, "mul_mat_glu: GLU op %d", glu_op);
    char reason[160];
    WView wg, wu;
    if (!mul_mat_ok(gate, src1, dst, true, &wg, reason, sizeof(reason)))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "mul_mat_glu: gate: %s", reason);
    if (!mul_mat_ok(up, src1, dst, true, &wu, reason, sizeof(reason)))
        return fail(ctx, QMM_ERR_UNSUPPORTED, "mul_mat_glu: up: %s", reason);
    if (memcmp(gate->ne, up->ne, sizeof(gate->ne))) return fail(ctx, QMM_ERR_INVALID, "mul_mat_glu: gate and up shapes differ");
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    if (up->type == gate->type) {                                 // one fused launch: gate, up and the GLU
        GemvDense dn;
        dn.ne11 = src1->ne[1];
        dn.ne12 = src1->ne[2];
        dn.ne13 = src1->ne[3];
        dn.r2 = src1->ne[2] / gate->ne[2];
        dn.r3 = src1->ne[3] / gate->ne[3];
        dn.ne02 = gate->ne[2];
        dn.d_nb1 = (int64_t)(dst->nb[1] / 4);
        dn.d_nb2 = (int64_t)(dst->nb[2] / 4);
        dn.d_nb3 = (int64_t)(dst->nb[3] / 4);
        int frc;
        if (try_fused_dense(ctx, gate, src1, wg, dn, (float *)((uint8_t *)dst->buffer->ptr + dst->offs), wu.base, glu_op, false, &frc)) {
            ctx->path = "glu-fused-gemv-fq";
            return frc;
        }
    }
    const int64_t M = gate->ne[1], N = src1->ne[1], ne12 = src1->ne[2], nb = src1->ne[2] * src1->ne[3];
    const size_t half = (size_t)(M * N * nb);
    int rc = ensure(ctx, &ctx->glu, &ctx->glu_cap, 2 * half * sizeof(float));
    if (rc) return rc;
    float * sg = (float *)ctx->glu, * su = sg + half;
    const int type = gate->type;
    const int nc = gemv_task_cols(type, N);
    GemvPlan plan;
    const bool fused = up->type == type && nb == 1 && !use_gemm_for(type, wg, N, nb) &&
                       gemv_plan(type, wg, nc, (N + nc - 1) / nc * 2, true, nc >= gemv_mma_min_cols(), &plan);
    if (fused) {
        GemvDense dn;
        dn.ne11 = N;
        dn.ne12 = 2;                                              // batch 0: gate, 1: up
        dn.ne13 = 1;
        dn.r2 = dn.r3 = 1;
        dn.ne02 = 2;
        dn.d_nb1 = M;
        dn.d_nb2 = M * N;
        dn.d_nb3 = 2 * M * N;
        dn.base2 = wu.base;
        dn.col_bs = 0;                                            // both read src1's columns
        ZeroJob z{ sg, M, 2 * N, N, 2, M, M * N, 2 * M * N, 0 };
        ActBuf a{};
        if ((rc = quantize_src1(ctx, type, src1, false, &a, plan.KS > 1 ? &z : nullptr))) return rc;
        KTime kt;
        const KTime * ktp;
        if ((rc = ktime_pair(ctx, &kt, &ktp))) return rc;
        QMM_HIP(ctx, launch_gemv(type, wg, plan, a, nullptr, nullptr, &dn, sg, ctx->sink, ctx->stream, ktp));
        if ((rc = ktime_done(ctx))) return rc;
        ctx->path = plan.mma ? "glu-fused-gemv-mfma" : "glu-fused-gemv";
    } else {
        qmm_buffer sb;
        sb.ptr = ctx->glu;
        sb.size = ctx->glu_cap;
        qmm_tensor t[2];
        for (int i = 0; i < 2; ++i) {
            t[i] = qmm_tensor{};
            t[i].type = QMM_TYPE_F32;
            t[i].ne[0] = M;
            t[i].ne[1] = N;
            t[i].ne[2] = src1->ne[2];
            t[i].ne[3] = src1->ne[3];
            t[i].nb[0] = 4;
            t[i].nb[1] = 4 * (size_t)M;
            t[i].nb[2] = t[i].nb[1] * (size_t)N;
            t[i].nb[3] = t[i].nb[2] * (size_t)src1->ne[2];
            t[i].buffer = &sb;
            t[i].offs = i * half * sizeof(float);
        }
        const bool outer = ctx->in_graph;                         // one quantization for both products
        if (!outer) {
            ctx->graph_gen++;
            ctx->in_graph = true;
        }
        rc = qmm_mul_mat(ctx, gate, src1, &t[0]);
        if (rc == QMM_OK) rc = qmm_mul_mat(ctx, up, src1, &t[1]);
        if (!outer) ctx->in_graph = false;
        if (rc) return rc;
        ctx->path = "glu-" + ctx->path;
    }
    GluArgs g;
    g.gate = sg;
    g.up = su;
    g.dst = (float *)((uint8_t *)dst->buffer->ptr + dst->offs);
    g.M = M;
    g.N = N;
    g.nb = nb;
    g.ne12 = ne12;
    g.d_nb1 = (int64_t)(dst->nb[1] / 4);
    g.d_nb2 = (int64_t)(dst->nb[2] / 4);
    g.d_nb3 = (int64_t)(dst->nb[3] / 4);
    QMM_HIP(ctx, launch_glu(glu_op, g, ctx->stream));
    return QMM_OK;
}

// Self-check for the tests (declared in qmm_internal.h, not part of the op ABI): the weight
// loads the GEMV launch of a qmm_mul_mat (id_n_used == 0: src0 of shape ne0, src1 [K, N,
// nbatch]) or of a qmm_mul_mat_id (id_n_used > 0: N tokens of id_n_used ids over ne0[2]
// experts, every task on the first and on the last expert) would make, planned as those entry
// points plan them and replayed on the host by gemv_extent.  out[8] = image bytes, lowest
// first byte, highest end byte, highest sink end, real loads, sink loads, bad loads, the
// stage's read extent.  No device is touched.  QMM_ERR_UNSUPPORTED when the product would run
// on the GEMM instead.
int64_t qmm_internal_quantize_tiled(qmm_ctx * ctx, const qmm_tensor * src1, int32_t type, void * out, int64_t cap) {
    if (!ctx || !src1 || !out || src1->type != QMM_TYPE_F32 || !type_layout(type)) return 0;
    const int64_t K = src1->ne[0], bk = vec_dot_type(type) == QMM_TYPE_Q8_K ? 256 : 32;
    if (K <= 0 || K % bk) return 0;
    ctx->key.valid = false;                                   // a fresh quantization
    TiledAct t;
    if (quantize_src1_tiled(ctx, type, src1, (K + 255) / 256, &t)) return 0;
    const bool kq = t.vdt == QMM_TYPE_Q8_K;
    const size_t a = tiled_a_bytes(t.ntiles, t.nblk), d = tiled_d_bytes(t.ntiles, kq ? t.nblk / 8 : t.nblk);
    const size_t sb = kq ? tiled_s_bytes(t.ntiles, t.nblk) : 0;
    if ((int64_t)(a + d + sb) > cap) return 0;
    uint8_t * o = (uint8_t *)out;
    hipError_t e = hipMemcpyAsync(o, t.A, a, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(o + a, t.D, d, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess && kq) e = hipMemcpyAsync(o + a + d, t.S, sb, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? (int64_t)(a + d + sb) : 0;
}

int qmm_internal_gemv_extent(int32_t type, const int64_t ne0[4], int64_t N, int64_t nbatch, int64_t id_n_used,
                             int64_t out[8]) {
    const TypeLayout * L = type_layout(type);
    ImageShape sh;
    if (!L || !out || N < 1 || nbatch < 1 || id_n_used < 0 || !image_shape(*L, ne0, &sh)) return QMM_ERR_INVALID;
    WView w{ nullptr, sh.M, sh.K, sh.bpr, sh.G, sh.ntiles, L->tg };
    GemvPlan plan;
    GemvExtent e[2];
    FusedPlan fp;
    // the fused kernel's loads are k_gemv's with one K slice: replayed through the same plan shape
    auto as_plan = [&](const FusedPlan & f) {
        plan = GemvPlan{};
        plan.nc = f.nc;
        plan.ntasks = f.ntasks;
        plan.W = f.W;
        plan.KS = f.KS;
        plan.spw = f.spw;
        plan.mma = false;
        plan.tw = 1;
        plan.cm = 8;
    };
    if (id_n_used == 0) {
        if (use_gemm_for(type, w, N, nbatch)) return QMM_ERR_UNSUPPORTED;
        const int nc = gemv_task_cols(type, N);
        const int64_t ntasks = (N + nc - 1) / nc * nbatch;
        if (fused_dense_plan(type, w, N, nbatch, &fp, true)) as_plan(fp);
        else if (!gemv_plan(type, w, nc, ntasks, true, nc >= gemv_mma_min_cols(), &plan)) return QMM_ERR_UNSUPPORTED;
        GemvDense dn;
        dn.ne11 = N;
        dn.ne12 = nbatch;
        dn.ne13 = 1;
        dn.r2 = nbatch / sh.nmat;
        dn.r3 = 1;
        dn.ne02 = sh.nmat;
        if (sh.nmat < 1 || nbatch % sh.nmat) return QMM_ERR_INVALID;
        if (!gemv_extent(type, w, plan, &dn, sh.nmat, 0, &e[0])) return QMM_ERR_INVALID;
        e[1] = e[0];
    } else {
        const int64_t n_as = sh.nmat, npairs = id_n_used * N;
        const int64_t max_tasks = route_max_tasks(npairs, n_as);
        const int nc = (int)std::min<int64_t>(kMaxTaskCols, npairs);
        if (fused_id_plan(type, w, id_n_used, N, &fp)) as_plan(fp);
        else if (!gemv_plan(type, w, nc, max_tasks, false, npairs >= 2 * n_as, &plan)) return QMM_ERR_UNSUPPORTED;
        for (int i = 0; i < 2; ++i)
            if (!gemv_extent(type, w, plan, nullptr, n_as, i ? (int)(n_as - 1) : 0, &e[i])) return QMM_ERR_INVALID;
    }
    out[0] = e[0].image_bytes;
    out[1] = std::min(e[0].real_lo, e[1].real_lo);
    out[2] = std::max(e[0].real_hi, e[1].real_hi);
    out[3] = std::max(e[0].sink_hi, e[1].sink_hi);
    out[4] = e[0].real_loads;
    out[5] = e[0].sink_loads;
    out[6] = e[0].bad + e[1].bad;
    out[7] = e[0].read_end;
    return QMM_OK;
}

int qmm_graph_compute(qmm_ctx * ctx, const qmm_node * nodes, int n_nodes) {
    if (!ctx || (!nodes && n_nodes)) return QMM_ERR_INVALID;
    ctx->graph_gen++;
    ctx->in_graph = true;
    int rc = QMM_OK;
    for (int i = 0; i < n_nodes && rc == QMM_OK; ++i) {
        const qmm_node & n = nodes[i];
        if (n.op == QMM_OP_MUL_MAT) rc = qmm_mul_mat(ctx, n.src0, n.src1, n.dst);
        else if (n.op == QMM_OP_MUL_MAT_ID) rc = qmm_mul_mat_id(ctx, n.src0, n.src1, n.ids, n.dst);
        else rc = fail(ctx, QMM_ERR_UNSUPPORTED, "graph node %d: unsupported op %d", i, n.op);
        // a node that writes over the cached activations' source invalidates them
        if (ctx->key.valid) {
            qmm_tensor src{};
            src.type = QMM_TYPE_F32;
            src.buffer = const_cast<qmm_buffer *>(ctx->key.buf);
            src.offs = ctx->key.offs;
            memcpy(src.ne, ctx->key.ne, sizeof(src.ne));
            memcpy(src.nb, ctx->key.nb, sizeof(src.nb));
            if (ranges_overlap(&src, n.dst)) ctx->key.valid = false;
        }
        if (ctx->rkey.valid && ranges_overlap(&ctx->rkey.ids, n.dst)) ctx->rkey.valid = false;
    }
    ctx->in_graph = false;
    return rc;
}

int qmm_dequantize(qmm_ctx * ctx, const qmm_tensor * src, const qmm_tensor * dst) {
    if (!ctx || !src || !dst || !dst->buffer) return fail(ctx, QMM_ERR_INVALID, "dequantize: null argument");
    char reason[160];
    WView w;
    if (!weight_image(src, true, &w, reason, sizeof(reason))) return fail(ctx, QMM_ERR_UNSUPPORTED, "dequantize: %s", reason);
    if (dst->type != QMM_TYPE_F32 || !contiguous(dst) || nelements(dst->ne) != nelements(src->ne) || !span_ok(dst))
        return fail(ctx, QMM_ERR_INVALID, "dequantize: dst must be contiguous f32 with as many elements, in its buffer");
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    float * y = (float *)((uint8_t *)dst->buffer->ptr + dst->offs);
    QMM_HIP(ctx, launch_dequant(src->type, w, src->ne[2] * src->ne[3], y, ctx->stream));
    return QMM_OK;
}

int qmm_quantize_act(qmm_ctx * ctx, int32_t act_type, const qmm_tensor * src, void * out, size_t out_size) {
    if (ctx && ctx->capturing) return fail(ctx, QMM_ERR_INVALID, "quantize_act: not while capturing (it synchronizes the stream)");
    if (!ctx || !check_f32(src) || !out) return fail(ctx, QMM_ERR_INVALID, "quantize_act: bad argument");
    if (act_type != QMM_TYPE_Q8_0 && act_type != QMM_TYPE_Q8_K) return fail(ctx, QMM_ERR_INVALID, "quantize_act: type");
    const int bs = act_block(act_type), bb = act_type == QMM_TYPE_Q8_0 ? 34 : 292;
    const int64_t K = src->ne[0], ncols = src->ne[1] * src->ne[2] * src->ne[3];
    if (K % bs) return fail(ctx, QMM_ERR_INVALID, "quantize_act: K %% %d != 0", bs);
    const size_t need = (size_t)(ncols * (K / bs)) * bb;
    if (out_size < need) return fail(ctx, QMM_ERR_INVALID, "quantize_act: out needs %zu bytes", need);
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    ctx->key.valid = false;
    ActBuf a;
    int rc = quantize_src1(ctx, act_type == QMM_TYPE_Q8_0 ? QMM_TYPE_Q4_0 : QMM_TYPE_Q4_K, src, true, &a);
    if (rc) return rc;
    void * tmp = nullptr;
    QMM_HIP(ctx, hipMalloc(&tmp, need));
    hipError_t e = launch_act_to_blocks(a, tmp, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(out, tmp, need, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(tmp);                                   // the copy's error, if any, is the one reported
    if (e != hipSuccess) return fail(ctx, QMM_ERR_DEVICE, "quantize_act: %s", hipGetErrorString(e));
    return QMM_OK;
}

// Waits for the stream, then reports what the kernels flagged since the last call: MUL_MAT_ID
// ids at or past n_as (their rows were written as zeros; ggml-cpu asserts on them, P02:105).
int qmm_synchronize(qmm_ctx * ctx) {
    if (ctx && ctx->capturing) return fail(ctx, QMM_ERR_INVALID, "synchronize: not while capturing (it synchronizes the stream)");
    if (!ctx) return QMM_ERR_INVALID;
    QMM_HIP(ctx, hipMemcpyAsync(ctx->hflags, ctx->dflags, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
    QMM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->hflags[0]) {
        ctx->hflags[0] = 0;
        QMM_HIP(ctx, hipMemsetAsync(ctx->dflags, 0, sizeof(int32_t), ctx->stream));
        QMM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        return fail(ctx, QMM_ERR_INVALID, "mul_mat_id: ids at or past the expert count were routed (their rows were "
                                          "written as zeros; ggml-cpu asserts on such ids)");
    }
    return QMM_OK;
}

int64_t qmm_downgrades(qmm_ctx * ctx, char * buf, size_t buf_len) {
    if (!ctx) return -1;
    int64_t total = ctx->dg_other;
    size_t at = 0;
    if (buf && buf_len) buf[0] = 0;
    auto line = [&](const char * key, int64_t n) {
        if (!buf || at + 1 >= buf_len) return;
        const int w = snprintf(buf + at, buf_len - at, "src=qmm %s\t%lld\n", key, (long long)n);
        if (w > 0) at = std::min(buf_len - 1, at + (size_t)w);
    };
    for (int i = 0; i < ctx->n_dg; ++i) {
        line(ctx->dg[i].key, ctx->dg[i].count);
        total += ctx->dg[i].count;
    }
    if (ctx->dg_other) line("other", ctx->dg_other);
    return total;
}

int qmm_kernel_timing(qmm_ctx * ctx, int enable) {
    if (ctx && ctx->capturing) return fail(ctx, QMM_ERR_INVALID, "kernel_timing: not while capturing (it synchronizes the stream)");
    if (!ctx || enable < 0 || enable > 2) return QMM_ERR_INVALID;
    QMM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    ctx->ktime = enable != 0;
    ctx->ktime_markers = enable == 2;
    ctx->ktime_stop = nullptr;
    ctx->kev_used = 0;
    return QMM_OK;
}

int64_t qmm_kernel_times(qmm_ctx * ctx, double * ms, int64_t cap) {
    if (!ctx || (cap > 0 && !ms)) return -1;
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return -1;
    const int64_t n = (int64_t)(ctx->kev_used / 2);
    for (int64_t i = 0; i < n && i < cap; ++i) {
        float t = 0.0f;
        if (hipEventElapsedTime(&t, ctx->kev[2 * i], ctx->kev[2 * i + 1]) != hipSuccess) return -1;
        ms[i] = t;
    }
    return n;
}

int qmm_kernel_time(qmm_ctx * ctx, double * total_ms, int64_t * launches) {
    if (ctx && ctx->capturing) return fail(ctx, QMM_ERR_INVALID, "kernel_time: not while capturing (it synchronizes the stream)");
    if (!ctx || !total_ms || !launches) return QMM_ERR_INVALID;
    QMM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    double t = 0.0;
    for (size_t i = 0; i + 1 < ctx->kev_used; i += 2) {
        float ms = 0.0f;
        QMM_HIP(ctx, hipEventElapsedTime(&ms, ctx->kev[i], ctx->kev[i + 1]));
        t += ms;
    }
    *total_ms = t;
    *launches = (int64_t)(ctx->kev_used / 2);
    return QMM_OK;
}

int qmm_capture_begin(qmm_ctx * ctx) {
    if (!ctx) return QMM_ERR_INVALID;
    if (ctx->capturing) return fail(ctx, QMM_ERR_INVALID, "capture_begin: already capturing");
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    ctx->ktime_stop = nullptr;
    QMM_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    ctx->capture_failed = false;
    return QMM_OK;
}

int qmm_capture_end(qmm_ctx * ctx, qmm_graph ** out) {
    if (!ctx || !out) return QMM_ERR_INVALID;
    *out = nullptr;
    if (!ctx->capturing) return fail(ctx, QMM_ERR_INVALID, "capture_end: not capturing");
    const bool failed = ctx->capture_failed;
    ctx->capturing = false;
    ctx->capture_failed = false;
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(ctx->stream, &g);      // ends it whatever happened meanwhile
    if (e != hipSuccess || failed) {
        if (g) (void)hipGraphDestroy(g);
        if (failed) {                                              // the first failure's status and reason
            const std::string why = ctx->capture_err;
            return fail(ctx, ctx->capture_code, "capture_end: an op failed while capturing: %s", why.c_str());
        }
        return fail(ctx, QMM_ERR_DEVICE, "hipStreamEndCapture: %s", hipGetErrorString(e));
    }
    qmm_graph * r = new qmm_graph();
    r->graph = g;
    r->device = ctx->device;
    r->ctx = ctx;
    r->scratch_gen = ctx->scratch_gen;
    const hipError_t ei = hipGraphInstantiate(&r->exec, g, nullptr, nullptr, 0);
    if (ei != hipSuccess) {
        (void)hipGraphDestroy(g);
        delete r;
        return fail(ctx, QMM_ERR_DEVICE, "hipGraphInstantiate: %s", hipGetErrorString(ei));
    }
    *out = r;
    return QMM_OK;
}

int qmm_graph_launch(qmm_ctx * ctx, const qmm_graph * graph) {
    if (!ctx || !graph) return QMM_ERR_INVALID;
    if (ctx->capturing) return fail(ctx, QMM_ERR_INVALID, "graph_launch: not while capturing");
    if (graph->device != ctx->device) return fail(ctx, QMM_ERR_INVALID, "graph_launch: the graph is of another device");
    if (graph->ctx != ctx) return fail(ctx, QMM_ERR_INVALID, "graph_launch: the graph was captured on another context");
    if (graph->scratch_gen != ctx->scratch_gen)
        return fail(ctx, QMM_ERR_INVALID, "graph_launch: an op outside the graph grew the context's scratch after the "
                                          "capture, so the graph's buffers are gone; capture again");
    QMM_HIP(ctx, hipSetDevice(ctx->device));
    QMM_HIP(ctx, hipGraphLaunch(graph->exec, ctx->stream));
    return QMM_OK;
}

void qmm_graph_free(qmm_graph * graph) {
    if (!graph) return;
    (void)hipSetDevice(graph->device);
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
}

int qmm_timer_begin(qmm_ctx * ctx) {
    if (!ctx) return QMM_ERR_INVALID;
    QMM_HIP(ctx, hipEventRecord(ctx->ev0, ctx->stream));
    return QMM_OK;
}

float qmm_timer_end(qmm_ctx * ctx) {
    if (!ctx || ctx->capturing) return -1.0f;
    if (hipEventRecord(ctx->ev1, ctx->stream) != hipSuccess || hipEventSynchronize(ctx->ev1) != hipSuccess) return -1.0f;
    float ms = -1.0f;
    if (hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1) != hipSuccess) return -1.0f;
    return ms;
}

}  // extern "C"
