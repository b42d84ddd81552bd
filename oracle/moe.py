"""TEST INFRASTRUCTURE ONLY: CPU restatement of the MoE router and combine.

The router is llama.cpp's softmax gating as the reference fuses it
(kernel_topk_moe_softmax_norm, contrib/llama.cpp/patches/0000-09-moe-routing-gemm-tiles.patch
lines 899-1000; the ggml op chain it replaces is matched at
0000-02-lowbit-iq-types.patch lines 786-821): per token the softmax of its
expert logits, the k largest probabilities in descending order with ties to the
lower expert, and their probabilities divided by their sum clamped to
[cmin, cmax].  The order is that of the float32 values exp(x - max) the
reference ranks (its p[j] = exp(p[j] - m) and `bv == gv ? bi : INT_MAX`,
lines 935-966 of that patch), so two distinct logits whose float32 exp is equal
tie and go to the lower expert; the weights are computed in float64 (the GPU's
float32 softmax agrees to ~1e-7 relative).  The combine is build_moe_ffn's MUL by the weights, the ADDs
over the k slots in slot order, then the shared expert times the sigmoid of its
gate, each in float32 with no fused multiply-add (numpy rounds every
operation).  Pinned by tests/test_oracle_moe.py against closed forms and brute
force.  Only tests/ may import this module.
"""
from __future__ import annotations

import numpy as np


def softmax(logits: np.ndarray) -> np.ndarray:
    """row-wise softmax in float64 of logits [T, n_expert]"""
    x = np.asarray(logits, np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def rank_values(logits: np.ndarray) -> np.ndarray:
    """the float32 exp(x - max) of each logit, the values the reference's router ranks"""
    x = np.asarray(logits, np.float32)
    return np.exp(x - x.max(axis=1, keepdims=True)).astype(np.float32)


def topk(logits: np.ndarray, k: int, cmin: float, cmax: float):
    """ids [T, k] (int32) and weights [T, k] (float64) of the router."""
    p = softmax(logits)
    r = rank_values(logits)
    T, n = p.shape
    # descending float32 probability, ties to the lower expert: sort on (-r, expert)
    order = np.lexsort((np.broadcast_to(np.arange(n), p.shape), -r), axis=1)
    ids = order[:, :k].astype(np.int32)
    w = np.take_along_axis(p, ids.astype(np.int64), axis=1)
    s = np.clip(w.sum(axis=1, keepdims=True), cmin, cmax)
    return ids, w / s


def combine(experts: np.ndarray, weights: np.ndarray, shared: np.ndarray | None = None,
            gate: np.ndarray | None = None) -> np.ndarray:
    """experts [T, k, M], weights [T, k], shared [T, M], gate [T] -> [T, M] (float32)."""
    e = np.asarray(experts, np.float32)
    w = np.asarray(weights, np.float32)
    y = e[:, 0, :] * w[:, 0:1]
    for j in range(1, e.shape[1]):
        y = y + e[:, j, :] * w[:, j:j + 1]
    if shared is not None:
        g = np.asarray(gate, np.float32)
        sg = (np.float32(1.0) / (np.float32(1.0) + np.exp(-g.astype(np.float64)).astype(np.float32)))
        y = y + np.asarray(shared, np.float32) * sg[:, None]
    return y.astype(np.float32)
