"""TEST INFRASTRUCTURE ONLY: CPU restatement of the GLU that follows an FFN's gate/up pair.

ggml's split GLU (GGML_OP_GLU with two tensors, ggml-cpu's ggml_vec_*glu_f32 scalar forms;
the reference runs it after its fused gate+up GEMV, glu.cl whose loops
contrib/llama.cpp/patches/0000-01-kquant-integer-dpas.patch:1350-1470 reshapes):
  REGLU        x > 0 ? x g : 0
  GEGLU        0.5 x (1 + tanh(sqrt(2/pi) x (1 + 0.044715 x^2))) g
  SWIGLU       x / (1 + exp(-x)) g
  GEGLU_ERF    0.5 x (1 + erf(x / sqrt(2))) g
  GEGLU_QUICK  x / (1 + exp(-1.702 x)) g
in float64 here (the GPU's fp32 agrees to ~1e-7 relative).  ggml-cpu builds with
GGML_GELU_FP16 evaluate GEGLU through a table at fp16-rounded x; that variant is not
restated (parity unpinned for it).  Pinned by tests/test_oracle_glu.py.  Only tests/ may
import this module.
"""
from __future__ import annotations

import math

import numpy as np

REGLU, GEGLU, SWIGLU, GEGLU_ERF, GEGLU_QUICK = 0, 1, 2, 4, 5


def act(op: int, x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float64)
    with np.errstate(over="ignore"):                  # exp(-x) = inf at large -x: the limit 0 is right
        return _act(op, x)


def _act(op: int, x: np.ndarray) -> np.ndarray:
    if op == REGLU:
        return np.where(x > 0, x, 0.0)
    if op == GEGLU:
        return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * x * (1.0 + 0.044715 * x * x)))
    if op == SWIGLU:
        return x / (1.0 + np.exp(-x))
    if op == GEGLU_ERF:
        erf = np.vectorize(math.erf)
        return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))
    if op == GEGLU_QUICK:
        return x / (1.0 + np.exp(-1.702 * x))
    raise ValueError(op)


def glu(op: int, gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """act(gate) * up in float64"""
    return act(op, gate) * np.asarray(up, np.float64)
