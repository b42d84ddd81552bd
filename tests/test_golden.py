"""The golden vectors of tests/golden/ (written by tests/golden/make_golden.py from the C
oracle): the oracle reproduces every one of them bit for bit.  They anchor the oracle against
regressions; tests/test_gpu_golden.py checks the HIP path against the same files."""
import glob
import os

import numpy as np
import pytest

GOLD = sorted(glob.glob(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_*.npz")))
M, K = 4, 512


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def qtype_of(orc, path):
    name = os.path.basename(path)[len("golden_"):-len(".npz")]
    return {v: k for k, v in orc.NAMES.items()}[name]


def test_all_types_have_vectors(orc):
    assert len(GOLD) == len(orc.NAMES)


@pytest.mark.parametrize("path", GOLD, ids=lambda p: os.path.basename(p))
def test_oracle_reproduces_golden(orc, path):
    g = load(path)
    qt = qtype_of(orc, path)
    same = lambda a, b: np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))
    assert same(orc.dequantize(qt, g["w"], M * K).reshape(M, K), g["deq"])
    assert same(np.concatenate([orc.quantize_act(qt, r) for r in g["x"]]), g["xq"])
    assert same(orc.mul_mat(qt, g["w"], M, K, g["x"], threads=1), g["y"])
    assert same(orc.mul_mat_id(qt, g["wid"], M, K, 3, g["xid"], g["ids"], threads=1), g["yid"])
    # the planted edge cases are there: a zero-scale block and one at the fp16 maximum
    assert not g["deq"][0, :32].any() or qt in (orc.Q4_K, orc.Q5_K, orc.Q6_K, orc.IQ4_XS)
    assert np.isfinite(g["y"]).all() and not g["yid"][1, 1].any()
