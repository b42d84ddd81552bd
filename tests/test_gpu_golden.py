"""The HIP path against the golden vectors of tests/golden/ (the C oracle's outputs, committed):
dequantization and the activation quantizers bit for bit, MUL_MAT and MUL_MAT_ID within the
parity bar, all through the C-ABI."""
import glob
import os
import sys

import numpy as np
import pytest

from conftest import rel_err
from arcint_amd import qmm

GOLD = sorted(glob.glob(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_*.npz")))
NAMES = {"Q4_0": qmm.Q4_0, "Q8_0": qmm.Q8_0, "Q4_K": qmm.Q4_K, "Q5_K": qmm.Q5_K, "Q6_K": qmm.Q6_K,
         "IQ4_NL": qmm.IQ4_NL, "IQ4_XS": qmm.IQ4_XS}
VDT = {qmm.Q4_0: qmm.Q8_0, qmm.Q8_0: qmm.Q8_0, qmm.IQ4_NL: qmm.Q8_0}
M, K = 4, 512
TOL = 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("path", GOLD, ids=lambda p: os.path.basename(p))
def test_hip_matches_golden(path):
    name = os.path.basename(path)[len("golden_"):-len(".npz")]
    print("[case] golden", name, flush=True)
    sys.stdout.flush()
    qt = NAMES[name]
    with np.load(path, allow_pickle=False) as z:
        g = {k: z[k] for k in z.files}
    with qmm.Backend(0) as be:
        bufs = []

        def new(qtype, ne, data=None):
            t = be.new_tensor(qtype, ne)
            bufs.append(t.buf)
            if data is not None:
                be.set_tensor(t, np.ascontiguousarray(data).view(np.uint8).ravel())
            return t

        w = new(qt, (K, M), g["w"])
        y = new(qmm.F32, (K, M))
        be.dequantize(w, y)
        be.synchronize()
        assert np.array_equal(be.get_tensor(y).view(np.uint32), g["deq"].ravel().view(np.uint32))
        xt = new(qmm.F32, (K, g["x"].shape[0]), g["x"].astype(np.float32))
        assert np.array_equal(be.quantize_act(VDT.get(qt, qmm.Q8_K), xt), g["xq"])
        for n in (1, g["x"].shape[0]):                       # the GEMV at one column, then all five
            xn = new(qmm.F32, (K, n), g["x"][:n].astype(np.float32))
            yn = new(qmm.F32, (M, n))
            be.mul_mat(w, xn, yn)
            be.synchronize()
            got = be.get_tensor(yn).view(np.float32).reshape(n, M)
            assert rel_err(got, g["y"][:n]) <= TOL
        wid = new(qt, (K, M, 3), g["wid"])
        xid = new(qmm.F32, (K, 1, 3), g["xid"].astype(np.float32))
        ids = new(qmm.I32, (2, 3), g["ids"].astype(np.int32))
        yid = new(qmm.F32, (M, 2, 3))
        be.mul_mat_id(wid, xid, ids, yid)
        be.synchronize()
        got = be.get_tensor(yid).view(np.float32).reshape(3, 2, M)
        assert rel_err(got, g["yid"]) <= TOL and not got[1, 1].any()
        for b in bufs:
            be.free_buffer(b)
