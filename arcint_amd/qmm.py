"""ctypes binding of libqmm (include/qmm.h), shaped like a ggml backend.

    be = Backend(0)                         # ggml_backend_*_init
    buf = be.alloc_buffer(n)                # ggml_backend_buft_alloc_buffer
    w = be.tensor(buf, Q4_K, (K, M))        # a ggml_tensor view in the buffer
    be.set_tensor(w, gguf_bytes)            # ggml_backend_tensor_set
    be.mul_mat(w, x, y)                     # GGML_OP_MUL_MAT
    be.mul_mat_id(w, x, ids, y)             # GGML_OP_MUL_MAT_ID
    be.graph_compute([...])                 # ggml_backend_graph_compute

There is no CPU fallback: without the built library or a HIP device every
entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# QMM_LIB names another build of the same library (the sanitizer and mutation builds of the tests)
LIB_PATH = os.environ.get("QMM_LIB") or os.path.join(_HERE, "libqmm.so")

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, IQ4_NL, IQ4_XS, I32 = 0, 1, 2, 8, 12, 13, 14, 15, 20, 23, 26
OP_MUL_MAT, OP_MUL_MAT_ID = 1, 2
GLU_REGLU, GLU_GEGLU, GLU_SWIGLU, GLU_GEGLU_ERF, GLU_GEGLU_QUICK = 0, 1, 2, 4, 5
QUANT_TYPES = (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS)

# every symbol include/qmm.h declares
EXPORTS = (
    "qmm_ctx_create", "qmm_ctx_free", "qmm_last_error", "qmm_buffer_alloc", "qmm_buffer_free",
    "qmm_buffer_size", "qmm_buffer_base", "qmm_tensor_alloc_size", "qmm_tensor_nbytes", "qmm_type_block",
    "qmm_tensor_set", "qmm_tensor_get", "qmm_supports_op", "qmm_mul_mat", "qmm_mul_mat_id",
    "qmm_graph_compute", "qmm_dequantize", "qmm_quantize_act", "qmm_synchronize", "qmm_downgrades",
    "qmm_last_path", "qmm_timer_begin", "qmm_timer_end", "qmm_buffer_copy", "qmm_kernel_timing",
    "qmm_kernel_time", "qmm_tensor_pack", "qmm_tensor_unpack", "qmm_describe_mul_mat", "qmm_moe_topk",
    "qmm_moe_combine", "qmm_mul_mat_glu", "qmm_mul_mat_id_glu", "qmm_mul_mat_noalloc", "qmm_kernel_times",
    "qmm_capture_begin", "qmm_capture_end", "qmm_graph_launch", "qmm_graph_free", "qmm_moe_ffn",
)
NOALLOC_SCRATCH_BYTES = 16 << 20     # QMM_NOALLOC_SCRATCH_BYTES


class QmmError(RuntimeError):
    pass


class CTensor(C.Structure):
    pass


CTensor._fields_ = [("type", C.c_int32), ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4),
                    ("buffer", C.c_void_p), ("offs", C.c_size_t), ("view_src", C.POINTER(CTensor)),
                    ("view_offs", C.c_size_t)]


class LaunchInfo(C.Structure):
    _fields_ = [("path", C.c_char * 32), ("workgroups", C.c_int64), ("threads", C.c_int32),
                ("cols_per_task", C.c_int32), ("tasks", C.c_int64), ("k_waves", C.c_int32),
                ("k_slices", C.c_int32), ("groups_per_wave", C.c_int32), ("lds_bytes", C.c_int64),
                ("tiles_per_wg", C.c_int32)]


class CNode(C.Structure):
    _fields_ = [("op", C.c_int32), ("src0", C.POINTER(CTensor)), ("src1", C.POINTER(CTensor)),
                ("ids", C.POINTER(CTensor)), ("dst", C.POINTER(CTensor))]


# qmm_moe_ffn_args, field for field
_TP = C.POINTER(CTensor)


class CMoeFfn(C.Structure):
    _fields_ = [("gate_exps", _TP), ("up_exps", _TP), ("down_exps", _TP), ("x", _TP), ("logits", _TP),
                ("cmin", C.c_float), ("cmax", C.c_float), ("ids", _TP), ("weights", _TP), ("shared_gate", _TP),
                ("shared_up", _TP), ("shared_down", _TP), ("shared_logit", _TP), ("glu_op", C.c_int32),
                ("dst", _TP)]


_lib = None


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise QmmError(f"{LIB_PATH} is not built; run python -m arcint_amd.build")
        L = C.CDLL(LIB_PATH)
        vp, sz, i32, i64 = C.c_void_p, C.c_size_t, C.c_int32, C.c_int64
        T = C.POINTER(CTensor)
        L.qmm_ctx_create.argtypes = [C.c_int, C.POINTER(vp)]
        L.qmm_ctx_free.argtypes = [vp]
        L.qmm_last_error.argtypes = [vp]
        L.qmm_last_error.restype = C.c_char_p
        L.qmm_last_path.argtypes = [vp]
        L.qmm_last_path.restype = C.c_char_p
        L.qmm_buffer_alloc.argtypes = [vp, sz, C.POINTER(vp)]
        L.qmm_buffer_free.argtypes = [vp, vp]
        L.qmm_buffer_size.argtypes = [vp]
        L.qmm_buffer_size.restype = sz
        L.qmm_buffer_base.argtypes = [vp]
        L.qmm_buffer_base.restype = vp
        L.qmm_tensor_alloc_size.argtypes = [i32, C.POINTER(i64)]
        L.qmm_tensor_alloc_size.restype = sz
        L.qmm_tensor_nbytes.argtypes = [i32, C.POINTER(i64)]
        L.qmm_tensor_nbytes.restype = sz
        L.qmm_type_block.argtypes = [i32, C.POINTER(sz)]
        L.qmm_tensor_set.argtypes = [vp, T, vp, sz, sz]
        L.qmm_tensor_get.argtypes = [vp, T, vp, sz, sz]
        L.qmm_supports_op.argtypes = [vp, i32, T, T, T, T, C.c_char_p, sz]
        L.qmm_mul_mat.argtypes = [vp, T, T, T]
        L.qmm_mul_mat_id.argtypes = [vp, T, T, T, T]
        L.qmm_mul_mat_noalloc.argtypes = [vp, T, T, T]
        L.qmm_moe_topk.argtypes = [vp, T, T, T, C.c_float, C.c_float]
        L.qmm_moe_combine.argtypes = [vp, T, T, T, T, T]
        L.qmm_moe_ffn.argtypes = [vp, C.POINTER(CMoeFfn)]
        L.qmm_mul_mat_glu.argtypes = [vp, T, T, T, T, C.c_int32]
        L.qmm_mul_mat_id_glu.argtypes = [vp, T, T, T, T, T, C.c_int32]
        L.qmm_graph_compute.argtypes = [vp, C.POINTER(CNode), C.c_int]
        L.qmm_dequantize.argtypes = [vp, T, T]
        L.qmm_quantize_act.argtypes = [vp, i32, T, vp, sz]
        L.qmm_synchronize.argtypes = [vp]
        L.qmm_downgrades.argtypes = [vp, C.c_char_p, sz]
        L.qmm_downgrades.restype = i64
        L.qmm_timer_begin.argtypes = [vp]
        L.qmm_timer_end.argtypes = [vp]
        L.qmm_timer_end.restype = C.c_float
        L.qmm_buffer_copy.argtypes = [vp, vp, sz, vp, sz, sz]
        L.qmm_kernel_timing.argtypes = [vp, C.c_int]
        L.qmm_kernel_time.argtypes = [vp, C.POINTER(C.c_double), C.POINTER(i64)]
        L.qmm_kernel_times.argtypes = [vp, C.POINTER(C.c_double), i64]
        L.qmm_kernel_times.restype = i64
        L.qmm_tensor_pack.argtypes = [i32, C.POINTER(i64), vp, vp, sz]
        L.qmm_describe_mul_mat.argtypes = [T, T, T, C.POINTER(LaunchInfo)]
        L.qmm_tensor_unpack.argtypes = [i32, C.POINTER(i64), vp, vp, sz]
        L.qmm_capture_begin.argtypes = [vp]
        L.qmm_capture_end.argtypes = [vp, C.POINTER(vp)]
        L.qmm_graph_launch.argtypes = [vp, vp]
        L.qmm_graph_free.argtypes = [vp]
        _lib = L
    return _lib


def _ne4(ne) -> tuple:
    ne = tuple(int(v) for v in ne)
    return ne + (1,) * (4 - len(ne))


def type_block(qtype: int) -> tuple[int, int]:
    bb = C.c_size_t(0)
    bl = load().qmm_type_block(qtype, C.byref(bb))
    if not bl:
        raise QmmError(f"unknown type {qtype}")
    return bl, bb.value


def nbytes(qtype: int, ne) -> int:
    arr = (C.c_int64 * 4)(*_ne4(ne))
    return load().qmm_tensor_nbytes(qtype, arr)


def alloc_size(qtype: int, ne) -> int:
    arr = (C.c_int64 * 4)(*_ne4(ne))
    return load().qmm_tensor_alloc_size(qtype, arr)


def describe_mul_mat(src0: "Tensor", src1: "Tensor", dst: "Tensor") -> dict:
    """The launch qmm_mul_mat would make for these shapes (host only)."""
    info = LaunchInfo()
    rc = load().qmm_describe_mul_mat(C.byref(src0.c), C.byref(src1.c), C.byref(dst.c), C.byref(info))
    if rc:
        raise QmmError(f"qmm_describe_mul_mat: status {rc}")
    return {f: (getattr(info, f).decode() if f == "path" else getattr(info, f)) for f, _ in LaunchInfo._fields_}


def pack(qtype: int, ne, gguf: np.ndarray) -> np.ndarray:
    """Device image of a whole tensor from its GGUF bytes (host only)."""
    arr = (C.c_int64 * 4)(*_ne4(ne))
    g = np.ascontiguousarray(gguf, np.uint8)
    out = np.empty(alloc_size(qtype, ne), np.uint8)
    rc = load().qmm_tensor_pack(qtype, arr, g.ctypes.data, out.ctypes.data, out.nbytes)
    if rc:
        raise QmmError(f"qmm_tensor_pack: status {rc}")
    return out


def unpack(qtype: int, ne, image: np.ndarray) -> np.ndarray:
    """GGUF bytes of a whole tensor from its device image (host only)."""
    arr = (C.c_int64 * 4)(*_ne4(ne))
    im = np.ascontiguousarray(image, np.uint8)
    out = np.empty(nbytes(qtype, ne), np.uint8)
    rc = load().qmm_tensor_unpack(qtype, arr, im.ctypes.data, out.ctypes.data, out.nbytes)
    if rc:
        raise QmmError(f"qmm_tensor_unpack: status {rc}")
    return out


@dataclass
class Buffer:
    ptr: int
    size: int


class Tensor:
    """A view {type, ne, nb, buffer, offs, view_src, view_offs}; nb defaults to the contiguous
    strides.  Views of a tensor come from Tensor.view, as ggml_view_* / ggml_permute /
    ggml_reshape make them."""

    def __init__(self, buf: Buffer, qtype: int, ne, offs: int = 0, nb=None, view_src: "Tensor | None" = None,
                 view_offs: int = 0):
        self.buf = buf
        self.type = qtype
        self.ne = _ne4(ne)
        bl, bb = type_block(qtype)
        if nb is None:
            nb = [bb, bb * (self.ne[0] // bl)]
            nb.append(nb[1] * self.ne[1])
            nb.append(nb[2] * self.ne[2])
        self.nb = tuple(int(v) for v in nb)
        self.offs = int(offs)
        self.view_src = view_src          # kept alive: the C struct points at its struct
        self.view_offs = int(view_offs)
        self.c = CTensor(qtype, (C.c_int64 * 4)(*self.ne), (C.c_size_t * 4)(*self.nb), buf.ptr, self.offs,
                         C.pointer(view_src.c) if view_src is not None else None, self.view_offs)

    def view(self, ne, nb=None, offset: int = 0) -> "Tensor":
        """ggml_view_4d: ne / nb (default contiguous) at byte `offset` of this tensor's layout;
        its base is this tensor's base."""
        base = self.view_src or self
        voff = self.view_offs + int(offset)
        return Tensor(self.buf, self.type, ne, self.offs + int(offset), nb, base, voff)

    @property
    def nbytes(self) -> int:
        """ggml_nbytes: first to past the last element, with the tensor's strides"""
        bl, _ = type_block(self.type)
        return self.ne[0] // bl * self.nb[0] + sum((n - 1) * s for n, s in zip(self.ne[1:], self.nb[1:]))


class Graph:
    """An instantiated capture (qmm_capture_end); free() it before its Backend closes."""

    def __init__(self, L, h):
        self.L = L
        self.h = h

    def free(self):
        if self.h:
            self.L.qmm_graph_free(self.h)
            self.h = None


class Backend:
    def __init__(self, device: int = 0):
        self.L = load()
        h = C.c_void_p()
        rc = self.L.qmm_ctx_create(device, C.byref(h))
        if rc != 0:
            raise QmmError(f"qmm_ctx_create({device}) failed with {rc}: no HIP device?")
        self.h = h
        self._bufs: list[Buffer] = []

    def close(self):
        if self.h:
            for b in self._bufs:
                self.L.qmm_buffer_free(self.h, C.c_void_p(b.ptr))
            self._bufs = []
            self.L.qmm_ctx_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc: int, what: str):
        if rc != 0:
            raise QmmError(f"{what}: status {rc}: {self.L.qmm_last_error(self.h).decode()}")

    # ---- memory ----
    def alloc_buffer(self, size: int) -> Buffer:
        p = C.c_void_p()
        self._check(self.L.qmm_buffer_alloc(self.h, size, C.byref(p)), "alloc_buffer")
        b = Buffer(p.value, size)
        self._bufs.append(b)
        return b

    def free_buffer(self, b: Buffer):
        self.L.qmm_buffer_free(self.h, C.c_void_p(b.ptr))
        self._bufs = [x for x in self._bufs if x.ptr != b.ptr]

    def tensor(self, buf: Buffer, qtype: int, ne, offs: int = 0, nb=None) -> Tensor:
        return Tensor(buf, qtype, ne, offs, nb)

    def new_tensor(self, qtype: int, ne) -> Tensor:
        """A contiguous tensor in a buffer of its own."""
        buf = self.alloc_buffer(alloc_size(qtype, ne))
        return Tensor(buf, qtype, ne)

    def set_tensor(self, t: Tensor, data, offset: int = 0):
        a = np.ascontiguousarray(data)
        self._check(self.L.qmm_tensor_set(self.h, C.byref(t.c), a.ctypes.data, offset, a.nbytes), "set_tensor")

    def get_tensor(self, t: Tensor, offset: int = 0, size: int | None = None) -> np.ndarray:
        size = t.nbytes - offset if size is None else size
        out = np.empty(size, np.uint8)
        self._check(self.L.qmm_tensor_get(self.h, C.byref(t.c), out.ctypes.data, offset, size), "get_tensor")
        return out

    def get_f32(self, t: Tensor) -> np.ndarray:
        return self.get_tensor(t).view(np.float32)

    # ---- ops ----
    def supports_op(self, op: int, src0: Tensor, src1: Tensor, ids: Tensor | None, dst: Tensor):
        buf = C.create_string_buffer(256)
        ok = self.L.qmm_supports_op(self.h, op, C.byref(src0.c), C.byref(src1.c),
                                    C.byref(ids.c) if ids else None, C.byref(dst.c), buf, 256)
        return bool(ok), buf.value.decode()

    def mul_mat(self, src0: Tensor, src1: Tensor, dst: Tensor):
        self._check(self.L.qmm_mul_mat(self.h, C.byref(src0.c), C.byref(src1.c), C.byref(dst.c)), "mul_mat")

    def mul_mat_noalloc(self, src0: Tensor, src1: Tensor, dst: Tensor):
        """qmm_mul_mat with the activations in the library's per-device array: allocates nothing"""
        self._check(self.L.qmm_mul_mat_noalloc(self.h, C.byref(src0.c), C.byref(src1.c), C.byref(dst.c)),
                    "mul_mat_noalloc")

    def mul_mat_id(self, src0: Tensor, src1: Tensor, ids: Tensor, dst: Tensor):
        self._check(self.L.qmm_mul_mat_id(self.h, C.byref(src0.c), C.byref(src1.c), C.byref(ids.c), C.byref(dst.c)),
                    "mul_mat_id")

    def mul_mat_glu(self, gate: Tensor, up: Tensor, src1: Tensor, dst: Tensor, op: int = GLU_SWIGLU):
        """dst = act(gate x src1) * (up x src1): MUL_MAT, MUL_MAT and the split GLU in one call"""
        self._check(self.L.qmm_mul_mat_glu(self.h, C.byref(gate.c), C.byref(up.c), C.byref(src1.c), C.byref(dst.c), op),
                    "mul_mat_glu")

    def mul_mat_id_glu(self, gate: Tensor, up: Tensor, src1: Tensor, ids: Tensor, dst: Tensor, op: int = GLU_SWIGLU):
        """dst = act(gate_experts x src1) * (up_experts x src1), routed by ids"""
        self._check(self.L.qmm_mul_mat_id_glu(self.h, C.byref(gate.c), C.byref(up.c), C.byref(src1.c), C.byref(ids.c),
                                              C.byref(dst.c), op), "mul_mat_id_glu")

    def moe_topk(self, logits: Tensor, ids: Tensor, weights: Tensor, cmin: float = 6.103515625e-5,
                 cmax: float = float("inf")):
        """Router: softmax over each token's expert logits, top-k ids and their clamped-sum
        normalized weights (cmin / cmax default to llama.cpp's clamp of the weight sum)."""
        self._check(self.L.qmm_moe_topk(self.h, C.byref(logits.c), C.byref(ids.c), C.byref(weights.c), cmin, cmax),
                    "moe_topk")

    def moe_combine(self, experts: Tensor, weights: Tensor, dst: Tensor, shared: Tensor | None = None,
                    gate: Tensor | None = None):
        """dst[:, t] = sum_j weights[j, t] experts[:, j, t] (+ shared[:, t] sigmoid(gate[0, t]))."""
        ref = lambda t: C.byref(t.c) if t is not None else None
        self._check(self.L.qmm_moe_combine(self.h, C.byref(experts.c), C.byref(weights.c), ref(shared), ref(gate),
                                           C.byref(dst.c)), "moe_combine")

    def moe_ffn(self, gate: Tensor, up: Tensor, down: Tensor, x: Tensor, ids: Tensor, weights: Tensor, dst: Tensor,
                shared: tuple | None = None, shared_logit: Tensor | None = None, op: int = GLU_SWIGLU,
                logits: Tensor | None = None, cmin: float = 6.103515625e-5, cmax: float = float("inf")):
        """A MoE FFN block in two launches: dst[:, t] = sum_j weights[j, t] down[ids[j, t]]
        glu(gate[ids[j, t]] x_t, up[ids[j, t]] x_t) (+ sigmoid(shared_logit[0, t]) sdown glu(sgate x_t,
        sup x_t) with shared = (sgate, sup, sdown)).  With logits the router runs inside and ids /
        weights are written (moe_topk's values)."""
        ptr = lambda t: C.pointer(t.c) if t is not None else None
        sg, su, sd = shared if shared is not None else (None, None, None)
        a = CMoeFfn(ptr(gate), ptr(up), ptr(down), ptr(x), ptr(logits), cmin, cmax, ptr(ids), ptr(weights), ptr(sg),
                    ptr(su), ptr(sd), ptr(shared_logit), op, ptr(dst))
        self._check(self.L.qmm_moe_ffn(self.h, C.byref(a)), "moe_ffn")

    def graph_compute(self, nodes):
        """nodes: list of (op, src0, src1, ids_or_None, dst)."""
        arr = (CNode * len(nodes))()
        for i, (op, s0, s1, ids, d) in enumerate(nodes):
            arr[i] = CNode(op, C.pointer(s0.c), C.pointer(s1.c), C.pointer(ids.c) if ids else None, C.pointer(d.c))
        self._check(self.L.qmm_graph_compute(self.h, arr, len(nodes)), "graph_compute")

    def capture_begin(self):
        """start recording the ops of this context's stream into a HIP graph (qmm_capture_begin)"""
        self._check(self.L.qmm_capture_begin(self.h), "capture_begin")

    def capture_end(self) -> "Graph":
        """end the recording; the instantiated graph (qmm_capture_end: raises if an op failed)"""
        g = C.c_void_p()
        self._check(self.L.qmm_capture_end(self.h, C.byref(g)), "capture_end")
        return Graph(self.L, g)

    def graph_launch(self, g: "Graph"):
        self._check(self.L.qmm_graph_launch(self.h, g.h), "graph_launch")

    def dequantize(self, src: Tensor, dst: Tensor):
        self._check(self.L.qmm_dequantize(self.h, C.byref(src.c), C.byref(dst.c)), "dequantize")

    def quantize_act(self, act_type: int, src: Tensor) -> np.ndarray:
        bs, bb = (32, 34) if act_type == Q8_0 else (256, 292)
        n = src.ne[0] // bs * src.ne[1] * src.ne[2] * src.ne[3] * bb
        out = np.empty(n, np.uint8)
        self._check(self.L.qmm_quantize_act(self.h, act_type, C.byref(src.c), out.ctypes.data, n), "quantize_act")
        return out

    def synchronize(self):
        self._check(self.L.qmm_synchronize(self.h), "synchronize")

    def downgrades(self) -> tuple[int, dict]:
        """(total count, {key: count}) of the ops that took a slower path than their type promises"""
        buf = C.create_string_buffer(1 << 14)
        n = self.L.qmm_downgrades(self.h, buf, len(buf))
        keys = {}
        for line in buf.value.decode().splitlines():
            k, _, c = line.rpartition("\t")
            keys[k] = int(c)
        return int(n), keys

    def last_path(self) -> str:
        return self.L.qmm_last_path(self.h).decode()

    def timer_begin(self):
        self._check(self.L.qmm_timer_begin(self.h), "timer_begin")

    def timer_end(self) -> float:
        ms = self.L.qmm_timer_end(self.h)
        if ms < 0:
            raise QmmError("timer_end failed")
        return ms

    def kernel_timing(self, enable, markers: bool = False):
        """start (enable) or stop stamping the ops' main kernels: dispatch stamps, or with
        markers event records on the stream around each launch"""
        self._check(self.L.qmm_kernel_timing(self.h, (2 if markers else 1) if enable else 0), "kernel_timing")

    def kernel_times(self) -> np.ndarray:
        """milliseconds of each main-kernel launch since kernel_timing(True)"""
        n = self.L.qmm_kernel_times(self.h, None, 0)
        if n < 0:
            raise QmmError("kernel_times failed")
        out = np.zeros(max(n, 1), np.float64)
        if self.L.qmm_kernel_times(self.h, out.ctypes.data_as(C.POINTER(C.c_double)), n) != n:
            raise QmmError("kernel_times failed")
        return out[:n]

    def kernel_time(self) -> tuple[float, int]:
        """(summed ms, launches) of the main kernels since kernel_timing(True)"""
        ms, n = C.c_double(0), C.c_int64(0)
        self._check(self.L.qmm_kernel_time(self.h, C.byref(ms), C.byref(n)), "kernel_time")
        return ms.value, n.value

    def copy(self, dst: Buffer, dst_off: int, src: Buffer, src_off: int, size: int):
        self._check(self.L.qmm_buffer_copy(self.h, C.c_void_p(dst.ptr), dst_off, C.c_void_p(src.ptr), src_off, size),
                    "buffer_copy")
