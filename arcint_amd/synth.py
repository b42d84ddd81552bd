"""Seeded synthetic GGUF weights and activations.

Distributions follow the benchmark definition of the reference's configs:
  Q4_0    d = fp16(|N(0, 0.02)|), codes U{0..15}
  Q8_0    d = fp16(|N(0, 0.02)|), codes U{-127..127}
  Q4_K    d, dmin = fp16(|N(0, 0.02)|), 12 scale bytes U{0..255}, code bytes U
  Q6_K    ql, qh U bytes, scales U{-128..127}, d = fp16(|N(0, 0.002)|)
  IQ4_XS  d = fp16(|N(0, 0.02)|), scales_h / scales_l / code bytes U
  Q5_K    as Q4_K, with qh bytes U
  IQ4_NL  as Q4_0 (the codes index the codebook)
  activations f32 N(0, 1); MoE ids = top-k of softmax(N(0, 1) logits)
Scales are made from floats, so no fp16 NaN or Inf ever appears.  Each tensor
takes its own numpy PCG64 stream (seed + a tensor index).
"""
from __future__ import annotations

import numpy as np

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, IQ4_NL, IQ4_XS = 2, 8, 12, 13, 14, 15, 20, 23
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), IQ4_NL: (32, 18),
         IQ4_XS: (256, 136)}
NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", IQ4_NL: "IQ4_NL", IQ4_XS: "IQ4_XS"}
BY_NAME = {v: k for k, v in NAMES.items()}


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(v.astype(np.float16)).view(np.uint8).reshape(v.shape + (2,))


def weights(qtype: int, rows: int, k: int, seed: int) -> np.ndarray:
    """GGUF bytes of a [rows, k] weight matrix, uint8 [rows * k / blck * bytes]."""
    blck, nbytes = BLOCK[qtype]
    assert k % blck == 0
    nb = rows * (k // blck)
    g = rng(seed)
    b = np.empty((nb, nbytes), np.uint8)
    if qtype in (Q4_0, IQ4_NL):
        b[:, 0:2] = _f16_bytes(np.abs(g.normal(0, 0.02, nb)).astype(np.float32))
        b[:, 2:] = g.integers(0, 256, (nb, 16), dtype=np.uint8)
    elif qtype == Q8_0:
        b[:, 0:2] = _f16_bytes(np.abs(g.normal(0, 0.02, nb)).astype(np.float32))
        b[:, 2:] = g.integers(-127, 128, (nb, 32), dtype=np.int8).view(np.uint8)
    elif qtype in (Q4_K, Q5_K):
        b[:, 0:2] = _f16_bytes(np.abs(g.normal(0, 0.02, nb)).astype(np.float32))
        b[:, 2:4] = _f16_bytes(np.abs(g.normal(0, 0.02, nb)).astype(np.float32))
        b[:, 4:] = g.integers(0, 256, (nb, nbytes - 4), dtype=np.uint8)
    elif qtype == Q6_K:
        b[:, 0:192] = g.integers(0, 256, (nb, 192), dtype=np.uint8)
        b[:, 192:208] = g.integers(-128, 128, (nb, 16), dtype=np.int8).view(np.uint8)
        b[:, 208:210] = _f16_bytes(np.abs(g.normal(0, 0.002, nb)).astype(np.float32))
    elif qtype == IQ4_XS:
        b[:, 0:2] = _f16_bytes(np.abs(g.normal(0, 0.02, nb)).astype(np.float32))
        b[:, 2:] = g.integers(0, 256, (nb, 134), dtype=np.uint8)
    else:
        raise ValueError(qtype)
    return b.reshape(-1)


def activations(n: int, k: int, seed: int) -> np.ndarray:
    return rng(seed).standard_normal((n, k), dtype=np.float32)


def moe_ids(tokens: int, n_expert: int, top_k: int, seed: int) -> np.ndarray:
    """int32 [tokens, top_k]: top-k of softmax over N(0, 1) router logits."""
    logits = rng(seed).standard_normal((tokens, n_expert), dtype=np.float32)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    return np.argsort(-p, axis=1, kind="stable")[:, :top_k].astype(np.int32)


def row_bytes(qtype: int, k: int) -> int:
    blck, nbytes = BLOCK[qtype]
    return k // blck * nbytes
