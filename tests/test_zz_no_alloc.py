"""qmm_mul_mat_noalloc (activations in the library's per-device array, nothing allocated)
against qmm_mul_mat on the same operands, through the C ABI, and against the CPU oracle: the GEMM
and both GEMV kernels, two and more calls in a row with the later ones smaller (the array keeps
the last call's contents), and a product whose activations need more than the array holds
(refused before anything runs)."""
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
