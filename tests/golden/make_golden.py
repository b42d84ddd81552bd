"""Writes the golden vectors of tests/golden/: per weight type, small seeded inputs and the C
oracle's outputs for them, as regression anchors (tests/test_golden.py checks the oracle still
reproduces them bit for bit; tests/test_gpu_golden.py checks the HIP path against them).

    python tests/golden/make_golden.py      # (after python -m arcint_amd.build)

Each golden_<TYPE>.npz holds
  w      uint8   GGUF bytes of a [4, 512] weight matrix (block 0 with a zero scale, block 1
                 with the fp16 maximum 65504 as its scale, where the type leads with an fp16 d)
  deq    float32 [4, 512]   dequantize_row of w
  x      float32 [5, 512]   activations (normal, all zero, quarter steps with exact ties, all
                 ones, one equal-magnitude pair of opposite signs)
  xq     uint8   the vec_dot type's quantization of x, row after row (q8_0 or q8_K blocks)
  y      float32 [5, 4]     MUL_MAT: x times w^T (ggml-cpu's numerics)
  wid    uint8   GGUF bytes of 3 experts [3][4][512]
  xid    float32 [3, 1, 512] tokens
  ids    int32   [3, 2]     expert ids (one -1: a zero row)
  yid    float32 [3, 2, 4]  MUL_MAT_ID
The inputs come from arcint_amd.synth with fixed seeds, but the files hold them, so the fixtures
do not depend on the generator staying the same.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from arcint_amd import synth  # noqa: E402

M, K, N, E, T, NU = 4, 512, 5, 3, 3, 2
# byte offset of the leading fp16 d in a block (Q6_K keeps d at the end)
D_OFF = {oracle.Q4_0: 0, oracle.Q8_0: 0, oracle.IQ4_NL: 0, oracle.Q4_K: 0, oracle.Q5_K: 0, oracle.IQ4_XS: 0,
         oracle.Q6_K: 208}


def special(qtype: int, raw: np.ndarray) -> np.ndarray:
    """block 0's scale set to +0, block 1's to the fp16 maximum (0x7bff)"""
    raw = raw.copy()
    _, nbytes = synth.BLOCK[qtype]
    o = D_OFF[qtype]
    raw[o:o + 2] = (0x00, 0x00)
    raw[nbytes + o:nbytes + o + 2] = (0xff, 0x7b)
    return raw


def acts(seed: int) -> np.ndarray:
    x = synth.activations(N, K, seed)
    x[1, :] = 0.0
    x[2, :] = np.round(x[2, :] * 4) / 4
    x[2, 0:K:32] = 127.0 / 4
    x[3, :] = 1.0
    x[4, 5], x[4, 100] = -9.0, 9.0
    return x


def make(qtype: int, seed: int) -> dict:
    w = special(qtype, synth.weights(qtype, M, K, seed))
    x = acts(seed + 1)
    wid = synth.weights(qtype, E * M, K, seed + 2)
    xid = synth.activations(T, K, seed + 3).reshape(T, 1, K)
    ids = np.array([[2, 0], [1, -1], [0, 2]], np.int32)
    return {
        "w": w,
        "deq": oracle.dequantize(qtype, w, M * K).reshape(M, K),
        "x": x,
        "xq": np.concatenate([oracle.quantize_act(qtype, r) for r in x]),
        "y": oracle.mul_mat(qtype, w, M, K, x, threads=1),
        "wid": wid,
        "xid": xid,
        "ids": ids,
        "yid": oracle.mul_mat_id(qtype, wid, M, K, E, xid, ids, threads=1),
    }


def main() -> None:
    for i, (qtype, name) in enumerate(sorted(oracle.NAMES.items())):
        d = make(qtype, 1000 + 10 * i)
        path = os.path.join(HERE, f"golden_{name}.npz")
        np.savez_compressed(path, **d)
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
