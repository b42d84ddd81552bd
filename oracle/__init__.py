"""TEST INFRASTRUCTURE ONLY: ctypes binding of the CPU oracle (liborc.so).

The oracle restates ggml's CPU arithmetic for MUL_MAT / MUL_MAT_ID on
Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K / IQ4_NL / IQ4_XS (see qmm_oracle.h for what pins each
function).  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg may import this package, and only as the checker or the timed CPU
baseline; the product path never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.environ.get("QMM_ORACLE_LIB") or os.path.join(_HERE, "liborc.so")   # (the sanitizer build: tests/sanitize.sh)

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, IQ4_NL, IQ4_XS = 2, 8, 12, 13, 14, 15, 20, 23
# type -> (weights per block, bytes per block, vec_dot type)
TYPES = {Q4_0: (32, 18, Q8_0), Q8_0: (32, 34, Q8_0), Q4_K: (256, 144, Q8_K), Q5_K: (256, 176, Q8_K),
         Q6_K: (256, 210, Q8_K), IQ4_NL: (32, 18, Q8_0), IQ4_XS: (256, 136, Q8_K)}
NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", IQ4_NL: "IQ4_NL",
         IQ4_XS: "IQ4_XS"}

_lib = None

# worker threads of mul_mat / mul_mat_id when the caller names none: the host share of a
# one-GPU box is 16 cores, whatever os.cpu_count() reports there
DEFAULT_THREADS = max(1, min(16, os.cpu_count() or 1))


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            raise FileNotFoundError(f"{_LIB} is not built (python -m arcint_amd.build)")
        L = C.CDLL(_LIB)
        vp, i64, f32p = C.c_void_p, C.c_int64, C.POINTER(C.c_float)
        L.orc_fp16_to_fp32.argtypes = [C.c_uint16]
        L.orc_fp16_to_fp32.restype = C.c_float
        L.orc_fp32_to_fp16.argtypes = [C.c_float]
        L.orc_fp32_to_fp16.restype = C.c_uint16
        L.orc_dequantize_row.argtypes = [C.c_int, vp, f32p, i64]
        L.orc_quantize_row_q8_0.argtypes = [f32p, vp, i64]
        L.orc_quantize_row_q8_K.argtypes = [f32p, vp, i64]
        L.orc_vec_dot.argtypes = [C.c_int, i64, vp, vp]
        L.orc_vec_dot.restype = C.c_float
        L.orc_mul_mat.argtypes = [C.c_int, vp, i64, i64, f32p, i64, f32p, C.c_int]
        L.orc_mul_mat_id.argtypes = [C.c_int, vp, i64, i64, i64, f32p, i64, C.POINTER(C.c_int32), i64, i64, f32p, C.c_int]
        L.orc_kvalues_iq4nl.restype = C.POINTER(C.c_int8)
        _lib = L
    return _lib


def _f32p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_float))


def fp16_to_fp32(h: int) -> float:
    return lib().orc_fp16_to_fp32(h)


def fp32_to_fp16(f: float) -> int:
    return lib().orc_fp32_to_fp16(f)


def kvalues() -> list[int]:
    p = lib().orc_kvalues_iq4nl()
    return [p[i] for i in range(16)]


def dequantize(qtype: int, raw: np.ndarray, k: int) -> np.ndarray:
    """raw: uint8 GGUF bytes of k weights -> float32 [k]."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    y = np.empty(k, np.float32)
    lib().orc_dequantize_row(qtype, raw.ctypes.data, _f32p(y), k)
    return y


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.zeros(x.size // 32 * 34, np.uint8)
    lib().orc_quantize_row_q8_0(_f32p(x), out.ctypes.data, x.size)
    return out


def quantize_q8_K(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.zeros(x.size // 256 * 292, np.uint8)
    lib().orc_quantize_row_q8_K(_f32p(x), out.ctypes.data, x.size)
    return out


def quantize_act(qtype: int, x: np.ndarray) -> np.ndarray:
    return quantize_q8_0(x) if TYPES[qtype][2] == Q8_0 else quantize_q8_K(x)


def vec_dot(qtype: int, k: int, w_row: np.ndarray, xq_row: np.ndarray) -> float:
    w_row = np.ascontiguousarray(w_row, np.uint8)
    xq_row = np.ascontiguousarray(xq_row, np.uint8)
    return lib().orc_vec_dot(qtype, k, w_row.ctypes.data, xq_row.ctypes.data)


def mul_mat(qtype: int, w: np.ndarray, M: int, K: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    """w: GGUF bytes of [M, K]; x: float32 [N, K] -> float32 [N, M]."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    N = x.shape[0]
    out = np.empty((N, M), np.float32)
    lib().orc_mul_mat(qtype, w.ctypes.data, M, K, _f32p(x), N, _f32p(out), threads or DEFAULT_THREADS)
    return out


def mul_mat_id(qtype: int, w: np.ndarray, M: int, K: int, E: int, x: np.ndarray, ids: np.ndarray,
               threads: int = 0) -> np.ndarray:
    """w: GGUF bytes [E][M][K]; x: float32 [T, ne11, K]; ids: int32 [T, n_used] -> [T, n_used, M]."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    T, ne11, _ = x.shape
    n_used = ids.shape[1]
    out = np.empty((T, n_used, M), np.float32)
    lib().orc_mul_mat_id(qtype, w.ctypes.data, M, K, E, _f32p(x), ne11,
                         ids.ctypes.data_as(C.POINTER(C.c_int32)), n_used, T, _f32p(out), threads or DEFAULT_THREADS)
    return out
