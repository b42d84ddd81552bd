"""qmm_mul_mat_noalloc (activations in the library's per-device array, nothing allocated)
against qmm_mul_mat on the same operands, through the C ABI, and against the CPU oracle, two and
more calls in a row with the later ones smaller (the array keeps the last call's contents).  Each
kernel path the entry point can take on the array is pinned by the path it reports:
  gemm-stream  the streaming GEMM (tiled pre-pass into the array)
  gemm-mfma    the shared-tile GEMM (the streaming kernels switched off: QMM_GEMM3_SBS=0, QMM_GEMM3=0)
  gemv-mfma    pre-pass + the few-column MFMA GEMV
  gemv         pre-pass + the v_dot4 GEMV: a large one-column product, which qmm_mul_mat runs as
               the K-split one-launch GEMV (its exchange-tree slots are allocated, so the
               allocation-free entry point takes the pre-pass path), and QMM_GEMV_FUSED=0
  gemv-fq      the one-launch GEMV of small products (no scratch at all)
plus a product whose activations need more than the array holds (refused before anything runs)
and a call with kernel timing on (the entry point records no timing events)."""
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


def product(be, qtype, M, K, N, seed):
    raw = synth.weights(qtype, M, K, seed)
    x = synth.activations(N, K, seed + 1)
    w = be.new_tensor(qtype, (K, M))
    be.set_tensor(w, raw)
    xt = be.new_tensor(qmm.F32, (K, N))
    be.set_tensor(xt, x.view(np.uint8).ravel())
    ya, yb = be.new_tensor(qmm.F32, (M, N)), be.new_tensor(qmm.F32, (M, N))
    return raw, x, w, xt, ya, yb


@pytest.mark.parametrize("seq", [
    # (type, M, K, N) in call order: each later call smaller than the first
    [(qmm.Q4_K, 4096, 4096, 512), (qmm.Q4_K, 1000, 2048, 3), (qmm.Q4_0, 300, 640, 1)],
    [(qmm.Q8_0, 2048, 11008, 64), (qmm.Q6_K, 512, 1024, 16), (qmm.IQ4_XS, 129, 256, 2)],
])
def test_noalloc_matches_mul_mat(be, orc, seq):
    for i, (qtype, M, K, N) in enumerate(seq):
        say("noalloc", i, synth.NAMES[qtype], M, K, N)
        raw, x, w, xt, ya, yb = product(be, qtype, M, K, N, seed=500 + 7 * i)
        be.mul_mat(w, xt, ya)
        path = be.last_path()
        be.mul_mat_noalloc(w, xt, yb)
        be.synchronize()
        assert be.last_path() == path
        a = be.get_f32(ya).reshape(N, M)
        b = be.get_f32(yb).reshape(N, M)
        assert rel_err(b, a) <= TOL, (i, path)
        assert rel_err(b, orc.mul_mat(qtype, raw, M, K, x)) <= TOL, (i, path)
        for t in (w, xt, ya, yb):
            be.free_buffer(t.buf)


@pytest.mark.parametrize("case", [
    # (type, M, K, N, environment, the path qmm_mul_mat_noalloc must report)
    (qmm.Q4_K, 17408, 5120, 1, {}, "gemv"),
    (qmm.Q4_K, 17408, 5120, 1, {"QMM_GEMV_FUSED": "0"}, "gemv"),
    (qmm.Q5_K, 1024, 2048, 64, {"QMM_GEMM3_SBS": "0"}, "gemm-mfma"),
    (qmm.Q4_0, 2048, 4096, 512, {"QMM_GEMM3": "0"}, "gemm-mfma"),
    (qmm.Q4_0, 2048, 4096, 512, {}, "gemm-stream"),
    (qmm.Q6_K, 4096, 2048, 512, {}, "gemm-stream"),
    (qmm.Q8_0, 4096, 4096, 24, {}, "gemv-mfma"),
    (qmm.IQ4_XS, 256, 512, 2, {}, "gemv-fq"),
    (qmm.Q6_K, 128, 256, 1, {}, "gemv-fq"),
])
def test_noalloc_paths(be, orc, monkeypatch, case):
    qtype, M, K, N, env, want = case
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    say("noalloc path", synth.NAMES[qtype], M, K, N, env, want)
    raw, x, w, xt, ya, yb = product(be, qtype, M, K, N, seed=700 + M % 97)
    be.mul_mat_noalloc(w, xt, yb)
    be.synchronize()
    assert be.last_path() == want
    be.mul_mat(w, xt, ya)
    be.synchronize()
    b = be.get_f32(yb).reshape(N, M)
    assert rel_err(b, be.get_f32(ya).reshape(N, M)) <= TOL
    assert rel_err(b, orc.mul_mat(qtype, raw, M, K, x)) <= TOL
    # a second, smaller call on the same array
    xs = qmm.Tensor(xt.buf, qmm.F32, (K, 1))
    ys = qmm.Tensor(yb.buf, qmm.F32, (M, 1))
    be.mul_mat_noalloc(w, xs, ys)
    be.synchronize()
    assert rel_err(be.get_f32(yb)[:M], orc.mul_mat(qtype, raw, M, K, x[:1])) <= TOL
    for t in (w, xt, ya, yb):
        be.free_buffer(t.buf)


def test_noalloc_records_no_timing(be, orc):
    """With kernel timing on, qmm_mul_mat stamps one event pair per op and the allocation-free
    entry point none, on every path (one-launch GEMV, pre-pass GEMV, GEMM)"""
    say("noalloc timing")
    cases = [(qmm.IQ4_XS, 256, 512, 2), (qmm.Q4_K, 2048, 4096, 1), (qmm.Q4_0, 2048, 4096, 512)]
    made = [(q, M, K, N, *product(be, q, M, K, N, seed=800 + i)) for i, (q, M, K, N) in enumerate(cases)]
    be.kernel_timing(1)
    try:
        for q, M, K, N, raw, x, w, xt, ya, yb in made:
            be.mul_mat_noalloc(w, xt, yb)
        be.synchronize()
        assert be.kernel_time()[1] == 0
        for q, M, K, N, raw, x, w, xt, ya, yb in made:
            be.mul_mat(w, xt, ya)
        assert be.kernel_time()[1] == len(made)
    finally:
        be.kernel_timing(0)
    for q, M, K, N, raw, x, w, xt, ya, yb in made:
        assert rel_err(be.get_f32(yb).reshape(N, M), orc.mul_mat(q, raw, M, K, x)) <= TOL
        for t in (w, xt, ya, yb):
            be.free_buffer(t.buf)


def test_noalloc_refuses_past_the_array(be):
    """K = 17408, N = 1024: about 20 MiB of quantized activations against the 16 MiB array -
    an error before any launch, dst untouched; the next call within the limit runs"""
    qtype, M, K, N = qmm.Q6_K, 64, 17408, 1024
    say("noalloc over the limit")
    raw, x, w, xt, ya, yb = product(be, qtype, M, K, N, seed=600)
    be.set_tensor(yb, np.full(M * N, 3.0, np.float32).view(np.uint8))
    with pytest.raises(qmm.QmmError, match="scratch"):
        be.mul_mat_noalloc(w, xt, yb)
    be.synchronize()
    assert (be.get_f32(yb) == 3.0).all()
    xs = qmm.Tensor(xt.buf, qmm.F32, (K, 4))                      # the first 4 columns
    ys = qmm.Tensor(yb.buf, qmm.F32, (M, 4))
    be.mul_mat_noalloc(w, xs, ys)
    be.mul_mat(w, xs, qmm.Tensor(ya.buf, qmm.F32, (M, 4)))
    be.synchronize()
    assert rel_err(be.get_f32(yb)[:4 * M], be.get_f32(ya)[:4 * M]) <= TOL
    for t in (w, xt, ya, yb):
        be.free_buffer(t.buf)
