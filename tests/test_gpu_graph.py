"""HIP-graph capture and replay (qmm_capture_begin / qmm_capture_end / qmm_graph_launch) through
the C ABI: a decode MoE layer (router, gate/up + SwiGLU, down, shared expert, combine) and dense
products on every MUL_MAT path, captured once and replayed several times with new inputs, with
the program's own eager work and synchronizations between the replays; every replay is checked
stage by stage against the CPU oracle.  Captures that would allocate or synchronize fail cleanly
and leave the stream usable."""
import sys

import numpy as np
import pytest

from arcint_amd import qmm, synth
from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def be():
    b = qmm.Backend(0)
    yield b
    b.close()


class Bufs:
    def __init__(self, be):
        self.be = be
        self.ts = []

    def weights(self, qtype, raw, ne):
        t = self.be.new_tensor(qtype, ne)
        self.be.set_tensor(t, raw)
        self.ts.append(t)
        return t

    def f32(self, arr):
        arr = np.ascontiguousarray(arr, np.float32)
        t = self.be.new_tensor(qmm.F32, tuple(reversed(arr.shape)))
        self.be.set_tensor(t, arr.view(np.uint8).ravel())
        self.ts.append(t)
        return t

    def empty(self, ne, qtype=qmm.F32):
        t = self.be.new_tensor(qtype, ne)
        self.ts.append(t)
        return t

    def close(self):
        for t in self.ts:
            self.be.free_buffer(t.buf)


@pytest.fixture
def bufs(be):
    b = Bufs(be)
    yield b
    b.close()


def put(be, t, arr):
    be.set_tensor(t, np.ascontiguousarray(arr, np.float32).view(np.uint8).ravel())


@pytest.mark.parametrize("T", [1, 4])
def test_graph_replay_moe_layer(be, orc, bufs, T):
    """router -> gate/up + SwiGLU -> down -> shared expert -> combine, captured once, replayed
    three times on new logits and activations"""
    from oracle import glu as G
    from oracle import moe
    E, k, HID, FFN, q = 64, 6, 1024, 256, qmm.Q4_K
    say("graph moe layer", T)
    raws = {n: synth.weights(q, r, c, 600 + i) for i, (n, r, c) in enumerate(
        [("gate", E * FFN, HID), ("up", E * FFN, HID), ("down", E * HID, FFN), ("sgate", FFN, HID),
         ("sup", FFN, HID), ("sdown", HID, FFN)])}
    wg = bufs.weights(q, raws["gate"], (HID, FFN, E))
    wu = bufs.weights(q, raws["up"], (HID, FFN, E))
    wd = bufs.weights(q, raws["down"], (FFN, HID, E))
    wsg = bufs.weights(q, raws["sgate"], (HID, FFN))
    wsu = bufs.weights(q, raws["sup"], (HID, FFN))
    wsd = bufs.weights(q, raws["sdown"], (FFN, HID))
    lt, xt, sgt = bufs.empty((E, T)), bufs.empty((HID, 1, T)), bufs.empty((1, T))
    xs = qmm.Tensor(xt.buf, qmm.F32, (HID, T))                   # the same activations as [HID, T]
    ids, wts = bufs.empty((k, T), qmm.I32), bufs.empty((k, T))
    h, ex = bufs.empty((FFN, k, T)), bufs.empty((HID, k, T))
    hs, ys, out = bufs.empty((FFN, T)), bufs.empty((HID, T)), bufs.empty((HID, T))
    other_w = bufs.weights(qmm.Q4_0, synth.weights(qmm.Q4_0, 128, 512, 690), (512, 128))
    other_x, other_y = bufs.f32(synth.activations(2, 512, 691)), bufs.empty((128, 2))

    def layer():
        be.moe_topk(lt, ids, wts)
        be.mul_mat_id_glu(wg, wu, xt, ids, h, qmm.GLU_SWIGLU)
        be.mul_mat_id(wd, qmm.Tensor(h.buf, qmm.F32, (FFN, k, T)), ids, ex)
        be.mul_mat_glu(wsg, wsu, xs, hs, qmm.GLU_SWIGLU)
        be.mul_mat(wsd, hs, ys)
        be.moe_combine(ex, wts, out, ys, sgt)

    def inputs(seed):
        g = np.random.default_rng(seed)
        logits = g.standard_normal((T, E)).astype(np.float32)
        x = synth.activations(T, HID, seed + 1)
        sgl = g.standard_normal((T, 1)).astype(np.float32)
        put(be, lt, logits)
        put(be, xt, x)
        put(be, sgt, sgl)
        return logits, x, sgl

    def check(logits, x, sgl, tag):
        got_ids = be.get_tensor(ids).view(np.int32).reshape(T, k)
        got_w = be.get_f32(wts).reshape(T, k)
        got_h = be.get_f32(h).reshape(T, k, FFN)
        got_ex = be.get_f32(ex).reshape(T, k, HID)
        got_hs = be.get_f32(hs).reshape(T, FFN)
        got_ys = be.get_f32(ys).reshape(T, HID)
        got = be.get_f32(out).reshape(T, HID)
        ref_ids, ref_w = moe.topk(logits, k, 6.103515625e-5, np.inf)
        assert np.array_equal(got_ids, ref_ids), tag
        np.testing.assert_allclose(got_w, ref_w, rtol=2e-6, atol=1e-30, err_msg=tag)
        xr = x.reshape(T, 1, HID)
        ref_h = G.glu(qmm.GLU_SWIGLU, orc.mul_mat_id(q, raws["gate"], FFN, HID, E, xr, ref_ids),
                      orc.mul_mat_id(q, raws["up"], FFN, HID, E, xr, ref_ids))
        assert rel_err(got_h, ref_h) <= TOL, tag
        assert rel_err(got_ex, orc.mul_mat_id(q, raws["down"], HID, FFN, E, got_h, ref_ids)) <= TOL, tag
        ref_hs = G.glu(qmm.GLU_SWIGLU, orc.mul_mat(q, raws["sgate"], FFN, HID, x),
                       orc.mul_mat(q, raws["sup"], FFN, HID, x))
        assert rel_err(got_hs, ref_hs) <= TOL, tag
        assert rel_err(got_ys, orc.mul_mat(q, raws["sdown"], HID, FFN, got_hs)) <= TOL, tag
        assert rel_err(got, moe.combine(got_ex, got_w, got_ys, sgl[:, 0])) <= TOL, tag

    ins = inputs(700)
    layer()                                                      # eager first: sizes the scratch
    be.synchronize()
    check(*ins, "eager")
    be.capture_begin()
    layer()
    g = be.capture_end()
    try:
        for r in range(3):
            ins = inputs(710 + 10 * r)
            be.graph_launch(g)
            be.synchronize()
            check(*ins, f"replay {r}")
            be.mul_mat(other_w, other_x, other_y)                # the program's own eager work between
            be.synchronize()
            assert rel_err(be.get_f32(other_y).reshape(2, 128),
                           orc.mul_mat(qmm.Q4_0, synth.weights(qmm.Q4_0, 128, 512, 690), 128, 512,
                                       synth.activations(2, 512, 691))) <= TOL
        ins = inputs(750)                                        # eager again after the replays
        layer()
        be.synchronize()
        check(*ins, "eager after")
    finally:
        g.free()


@pytest.mark.parametrize("qtype,M,K,N", [(qmm.Q4_K, 1000, 2048, 1), (qmm.Q4_K, 1000, 2048, 3),
                                         (qmm.Q4_K, 1000, 2048, 300), (qmm.Q4_0, 700, 4096, 1),
                                         (qmm.Q6_K, 512, 1024, 40), (qmm.Q4_0, 2048, 4096, 512)])
def test_graph_replay_mul_mat(be, orc, bufs, qtype, M, K, N):
    """one MUL_MAT captured (GEMV with split-K atomics into pre-pass-zeroed dst, the few-column
    MFMA GEMV, the streaming and the shared-tile GEMM), replayed with new activations"""
    say("graph mul_mat", synth.NAMES[qtype], M, K, N)
    raw = synth.weights(qtype, M, K, 800)
    w = bufs.weights(qtype, raw, (K, M))
    xt, y = bufs.empty((K, N)), bufs.empty((M, N))
    x = synth.activations(N, K, 801)
    put(be, xt, x)
    be.mul_mat(w, xt, y)                                         # eager first: sizes the scratch
    be.synchronize()
    path = be.last_path()
    assert rel_err(be.get_f32(y).reshape(N, M), orc.mul_mat(qtype, raw, M, K, x)) <= TOL
    be.capture_begin()
    be.mul_mat(w, xt, y)
    g = be.capture_end()
    try:
        for r in range(3):
            x = synth.activations(N, K, 810 + r)
            put(be, xt, x)
            be.graph_launch(g)
            be.synchronize()
            assert be.last_path() == path
            assert rel_err(be.get_f32(y).reshape(N, M), orc.mul_mat(qtype, raw, M, K, x)) <= TOL, (path, r)
    finally:
        g.free()


def test_capture_refuses_allocation(orc):
    """a fresh context has no scratch: the captured op (three columns over 16 groups along K:
    the pre-pass path, whose activations go to the scratch) fails, capture_end reports it, and
    the stream runs the same op eagerly afterwards"""
    say("graph capture needs scratch")
    with qmm.Backend(0) as b:
        qtype, M, K, N = qmm.Q4_K, 256, 4096, 3
        raw = synth.weights(qtype, M, K, 820)
        x = synth.activations(N, K, 821)
        w = b.new_tensor(qtype, (K, M))
        b.set_tensor(w, raw)
        xt = b.new_tensor(qmm.F32, (K, N))
        b.set_tensor(xt, x.view(np.uint8).ravel())
        y = b.new_tensor(qmm.F32, (M, N))
        b.capture_begin()
        with pytest.raises(qmm.QmmError):
            b.mul_mat(w, xt, y)
        with pytest.raises(qmm.QmmError, match="capture_end"):
            b.capture_end()
        b.capture_begin()
        with pytest.raises(qmm.QmmError, match="not while capturing"):
            b.synchronize()
        with pytest.raises(qmm.QmmError):
            b.capture_end()
        b.mul_mat(w, xt, y)
        b.synchronize()
        assert rel_err(b.get_f32(y).reshape(N, M), orc.mul_mat(qtype, raw, M, K, x)) <= TOL
        for t in (w, xt, y):
            b.free_buffer(t.buf)


def test_graph_refused_after_scratch_grows(be, orc):
    """an op outside a graph that needs more scratch than the context has replaces it: the graph
    captured before then is refused (its buffers are gone) and a new capture runs; a graph is
    refused on another context too"""
    say("graph refused after the scratch grows")
    with qmm.Backend(0) as b:
        qtype, M = qmm.Q4_K, 256
        ts = []

        def product(K, N, seed):
            raw = synth.weights(qtype, M, K, seed)
            x = synth.activations(N, K, seed + 1)
            w = b.new_tensor(qtype, (K, M))
            b.set_tensor(w, raw)
            xt = b.new_tensor(qmm.F32, (K, N))
            b.set_tensor(xt, x.view(np.uint8).ravel())
            y = b.new_tensor(qmm.F32, (M, N))
            ts.extend([w, xt, y])
            return raw, x, w, xt, y

        # 16 groups along K, 3 columns: the pre-pass path (activations in the scratch)
        raw, x, w, xt, y = product(4096, 3, 830)
        b.mul_mat(w, xt, y)
        b.synchronize()
        b.capture_begin()
        b.mul_mat(w, xt, y)
        g = b.capture_end()
        try:
            b.graph_launch(g)
            b.synchronize()
            assert rel_err(b.get_f32(y).reshape(3, M), orc.mul_mat(qtype, raw, M, 4096, x)) <= TOL
            with pytest.raises(qmm.QmmError, match="another context"):
                be.graph_launch(g)
            rb, xb, wb, xtb, yb = product(16384, 8, 840)          # more activations: the scratch grows
            b.mul_mat(wb, xtb, yb)
            b.synchronize()
            assert rel_err(b.get_f32(yb).reshape(8, M), orc.mul_mat(qtype, rb, M, 16384, xb)) <= TOL
            with pytest.raises(qmm.QmmError, match="capture again"):
                b.graph_launch(g)
        finally:
            g.free()
        b.capture_begin()
        b.mul_mat(w, xt, y)
        g2 = b.capture_end()
        try:
            b.graph_launch(g2)
            b.synchronize()
            assert rel_err(b.get_f32(y).reshape(3, M), orc.mul_mat(qtype, raw, M, 4096, x)) <= TOL
        finally:
            g2.free()
        for t in ts:
            b.free_buffer(t.buf)
