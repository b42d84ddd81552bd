"""GPU parity: libqmm on the HIP device against the CPU oracle, through the C ABI.

Bars: dequantization and activation quantization bit-exact (byte equality);
set_tensor / get_tensor byte-exact; MUL_MAT / MUL_MAT_ID within a max
relative error of 1e-3 in fp32 (denominator floored at 5 % of the output
rms, see conftest.rel_err) - the integer dots are exact on both sides, the
expected error is ~1e-6.  Each case prints its name first so that a fault
names it."""
import sys

import numpy as np
import pytest

from arcint_amd import qmm, synth
from conftest import rel_err

pytestmark = pytest.mark.gpu

TYPES = [qmm.Q4_0, qmm.Q8_0, qmm.Q4_K, qmm.Q5_K, qmm.Q6_K, qmm.IQ4_NL, qmm.IQ4_XS]
# the types whose 3..8-column products run on the MFMA GEMV
MMA_TYPES = (qmm.Q4_0, qmm.Q8_0, qmm.Q4_K, qmm.IQ4_XS, qmm.IQ4_NL, qmm.Q6_K)
TOL = 1e-3
# the types whose GEMM streams weights per wave (one float scale per 32-weight block)
STREAM_TYPES = (qmm.Q4_0, qmm.Q8_0, qmm.IQ4_NL, qmm.Q4_K, qmm.Q6_K, qmm.Q5_K, qmm.IQ4_XS)


def gemm_path(qtype):
    return "gemm-stream" if qtype in STREAM_TYPES else "gemm-mfma"


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def be():
    b = qmm.Backend(0)
    yield b
    b.close()


class Scope:
    """Buffers allocated for one test, freed at its end."""

    def __init__(self, be):
        self.be = be
        self.bufs = []

    def weights(self, qtype, raw, ne):
        t = self.be.new_tensor(qtype, ne)
        self.bufs.append(t.buf)
        self.be.set_tensor(t, raw)
        return t

    def f32(self, arr):
        arr = np.ascontiguousarray(arr, np.float32)
        t = self.be.new_tensor(qmm.F32, tuple(reversed(arr.shape)))
        self.bufs.append(t.buf)
        self.be.set_tensor(t, arr.view(np.uint8).ravel())
        return t

    def i32(self, arr):
        arr = np.ascontiguousarray(arr, np.int32)
        t = self.be.new_tensor(qmm.I32, tuple(reversed(arr.shape)))
        self.bufs.append(t.buf)
        self.be.set_tensor(t, arr.view(np.uint8).ravel())
        return t

    def empty_f32(self, ne):
        t = self.be.new_tensor(qmm.F32, ne)
        self.bufs.append(t.buf)
        return t

    def close(self):
        for b in self.bufs:
            self.be.free_buffer(b)


@pytest.fixture
def sc(be):
    s = Scope(be)
    yield s
    s.close()


def special_blocks(qtype, nblk, seed):
    """random blocks with some scales set to 0, the smallest subnormal and the fp16 max"""
    blck, bb = synth.BLOCK[qtype]
    raw = synth.weights(qtype, 1, blck * nblk, seed).reshape(nblk, bb).copy()
    doff = 208 if qtype == qmm.Q6_K else 0
    for i, bits in enumerate([0x0000, 0x8000, 0x0001, 0x7BFF, 0x03FF, 0xFBFF]):
        raw[i, doff:doff + 2] = np.frombuffer(np.uint16(bits).tobytes(), np.uint8)
        if qtype in (qmm.Q4_K, qmm.Q5_K):
            raw[i, 2:4] = np.frombuffer(np.uint16(bits).tobytes(), np.uint8)
    return raw.ravel()


# ------------------------------------------------------------------ memory
@pytest.mark.parametrize("qtype", TYPES)
def test_set_get_roundtrip(be, sc, qtype):
    say("set_get", qtype)
    blck, bb = synth.BLOCK[qtype]
    K, M = blck * 4, 37
    raw = synth.weights(qtype, M, K, seed=21)
    w = sc.weights(qtype, raw, (K, M))
    assert np.array_equal(be.get_tensor(w), raw)
    # partial writes and reads at block granularity
    part = synth.weights(qtype, 1, blck * 7, seed=22)
    be.set_tensor(w, part, offset=bb * 11)
    raw2 = raw.copy()
    raw2[bb * 11:bb * 18] = part
    assert np.array_equal(be.get_tensor(w), raw2)
    assert np.array_equal(be.get_tensor(w, offset=bb * 5, size=bb * 20), raw2[bb * 5:bb * 25])
    with pytest.raises(qmm.QmmError):                  # past the tensor's bytes
        be.set_tensor(w, part[:bb + 1], offset=raw.size - bb)


@pytest.mark.parametrize("qtype", TYPES)
def test_gguf_load_chunked(be, sc, orc, tmp_path, qtype):
    """a GGUF tensor streamed into the device image in chunks of a few whole blocks (chunk
    boundaries inside rows and across 64-row tiles) reads back as the file's bytes and
    multiplies like the oracle"""
    import gguf_writer
    from arcint_amd import gguf
    say("gguf_load", qtype)
    blck, bb = synth.BLOCK[qtype]
    M, K, N = 131, 1024, 5
    raw = synth.weights(qtype, M, K, seed=61)
    p = tmp_path / "w.gguf"
    gguf_writer.write(p, [("general.architecture", gguf_writer.STRING, "test")],
                      [("pad", (7,), qmm.F32, np.zeros(28, np.uint8)), ("blk.0.w", (K, M), qtype, raw)])
    g = gguf.read(str(p))
    w = gguf.load_tensor(be, g, "blk.0.w", chunk_bytes=7 * bb + 5)
    sc.bufs.append(w.buf)
    assert np.array_equal(be.get_tensor(w), raw)
    x = synth.activations(N, K, 62)
    xt = sc.f32(x)
    y = sc.empty_f32((M, N))
    be.mul_mat(w, xt, y)
    be.synchronize()
    assert rel_err(be.get_f32(y).reshape(N, M), orc.mul_mat(qtype, raw, M, K, x)) <= TOL


# ------------------------------------------------------------------ views and partial ranges
# The cases of the reference's tests/test_planes.cpp:106-286 (set_tensor / get_tensor of views
# go through the base; any byte range is exact), on the device image.
VK = 512


def dequant_matches(be, sc, orc, qtype, t, raw):
    """the device image of t decodes to the oracle's dequantization of raw (NaN where both are)"""
    n = int(np.prod(t.ne))
    y = sc.empty_f32(t.ne)
    be.dequantize(t, y)
    be.synchronize()
    return np.array_equal(be.get_f32(y), orc.dequantize(qtype, raw, n), equal_nan=True)


@pytest.mark.parametrize("qtype", TYPES)
def test_permuted_view_writes_through_its_base(be, sc, orc, qtype):
    say("view_permuted", qtype)
    M = 40
    raw = synth.weights(qtype, M, VK, seed=71)
    a = sc.weights(qtype, np.zeros_like(raw), (VK, 1, M))             # [K, 1, M]: M one-row matrices
    ap = a.view((VK, M), nb=(a.nb[0], a.nb[2], a.nb[2], M * a.nb[2]))   # permute(0, 2, 1, 3)
    assert ap.nbytes == a.nbytes
    be.set_tensor(ap, raw)
    assert np.array_equal(be.get_tensor(a), raw)
    assert np.array_equal(be.get_tensor(ap), raw)
    assert dequant_matches(be, sc, orc, qtype, a, raw)                # the image is the base's


@pytest.mark.parametrize("qtype", TYPES)
def test_partial_range_is_read_modify_write(be, sc, orc, qtype):
    say("partial_range", qtype)
    M = 6
    raw = synth.weights(qtype, M, VK, seed=72)
    a = sc.weights(qtype, raw, (VK, M))
    n = raw.size
    g = np.random.default_rng(73)
    exp = raw.copy()
    for at, ln in [(n // 2 + 7, 300), (5, 3), (0, 1), (n - 1, 1), (n - 301, 301), (1, n - 2)]:
        patch = g.integers(0, 256, ln, dtype=np.uint8)
        be.set_tensor(a, patch, offset=at)
        exp[at:at + ln] = patch
        assert np.array_equal(be.get_tensor(a), exp), (at, ln)
    assert np.array_equal(be.get_tensor(a, offset=41, size=123), exp[41:164])
    assert np.array_equal(be.get_tensor(a, offset=n - 5, size=5), exp[n - 5:])
    assert be.get_tensor(a, offset=7, size=0).size == 0
    assert dequant_matches(be, sc, orc, qtype, a, exp)
    with pytest.raises(qmm.QmmError):
        be.set_tensor(a, exp[:10], offset=n - 9)                       # past the tensor


@pytest.mark.parametrize("qtype", TYPES)
def test_reshape_of_a_3d_base_converts_by_the_base_slices(be, sc, orc, qtype):
    say("view_reshape", qtype)
    N, E = 64, 3
    raw = synth.weights(qtype, N * E, VK, seed=74)
    a = sc.weights(qtype, np.zeros_like(raw), (VK, N, E))
    a2 = a.view((VK, N * E))                                          # ggml_reshape_2d
    be.set_tensor(a2, raw)
    rows = a.view((VK, 5), offset=70 * a.nb[1])                       # rows 70..74: slice 1
    patch = synth.weights(qtype, 5, VK, seed=75)
    be.set_tensor(rows, patch)
    exp = raw.copy()
    exp[70 * a.nb[1]:75 * a.nb[1]] = patch
    assert np.array_equal(be.get_tensor(a), exp)
    assert np.array_equal(be.get_tensor(rows), patch)
    assert dequant_matches(be, sc, orc, qtype, a, exp)


@pytest.mark.parametrize("qtype", TYPES)
def test_partial_range_across_a_slice_boundary_is_exact(be, sc, orc, qtype):
    say("range_across_slices", qtype)
    raw = synth.weights(qtype, 4 * 3, VK, seed=76)
    a = sc.weights(qtype, raw, (VK, 4, 3))
    sb = a.nb[2]
    at, ln = sb - 37, sb + 100                                        # slice 0's tail .. slice 2's head
    patch = np.random.default_rng(77).integers(0, 256, ln, dtype=np.uint8)
    be.set_tensor(a, patch, offset=at)
    exp = raw.copy()
    exp[at:at + ln] = patch
    assert np.array_equal(be.get_tensor(a), exp)
    assert np.array_equal(be.get_tensor(a, offset=2 * sb - 40, size=80), exp[2 * sb - 40:2 * sb + 40])
    # the same through a view of slice 1: its range is its base's at view_offs
    s1 = a.view((VK, 4), offset=sb)
    assert np.array_equal(be.get_tensor(s1, offset=3, size=sb - 6), exp[sb + 3:2 * sb - 3])
    assert dequant_matches(be, sc, orc, qtype, a, exp)


def mul_mat_of(be, sc, w, K, N, seed):
    x = synth.activations(N * w.ne[2], K, seed)
    xt = sc.f32(x.reshape(w.ne[2], N, K))
    y = sc.empty_f32((w.ne[1], N, w.ne[2]))
    be.mul_mat(w, xt, y)
    be.synchronize()
    return x, be.get_f32(y).reshape(w.ne[2], N, w.ne[1])


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("N", [1, 5, 20])
def test_whole_slice_views_multiply_as_their_bytes(be, sc, orc, qtype, N):
    """views the image addresses (a slice, a run of slices, a reshape over whole tiles, rows
    64.. of a matrix) multiply like the oracle on the bytes they view"""
    say("view_mul_mat", qtype, N)
    blck, bb = synth.BLOCK[qtype]
    row = VK // blck * bb
    raw = synth.weights(qtype, 64 * 3, VK, seed=78)
    a = sc.weights(qtype, raw, (VK, 64, 3))
    big = synth.weights(qtype, 256, VK, seed=79)
    c = sc.weights(qtype, big, (VK, 256))
    cases = [(a.view((VK, 64), offset=2 * a.nb[2]), raw[2 * 64 * row:3 * 64 * row], 64),
             (a.view((VK, 64, 2), offset=a.nb[2]), None, 64),
             (a.view((VK, 192)), raw, 192),
             (c.view((VK, 128), offset=64 * row), big[64 * row:192 * row], 128)]
    for i, (v, vb, M) in enumerate(cases):
        x, got = mul_mat_of(be, sc, v, VK, N, seed=80 + i)
        if vb is not None:
            ref = orc.mul_mat(qtype, vb, M, VK, x)
            assert rel_err(got.reshape(N, M), ref) <= TOL, i
        else:                                                         # two slices, each its own matrix
            for j in range(2):
                vb = raw[(1 + j) * 64 * row:(2 + j) * 64 * row]
                ref = orc.mul_mat(qtype, vb, 64, VK, x[j * N:(j + 1) * N])
                assert rel_err(got[j], ref) <= TOL, (i, j)
    with pytest.raises(qmm.QmmError):                                 # rows 5..68: not whole tiles
        mul_mat_of(be, sc, a.view((VK, 64), offset=5 * row), VK, N, seed=90)


@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.IQ4_XS])
def test_mul_mat_id_on_a_run_of_experts(be, sc, orc, qtype):
    say("view_mul_mat_id", qtype)
    blck, bb = synth.BLOCK[qtype]
    M, E, T, k = 64, 8, 6, 2
    mat = M * VK // blck * bb
    raw = synth.weights(qtype, M * E, VK, seed=91)
    e = sc.weights(qtype, raw, (VK, M, E))
    ev = e.view((VK, M, 4), offset=3 * e.nb[2])                       # experts 3..6 as 0..3
    g = np.random.default_rng(92)
    ids = np.stack([g.permutation(4)[:k] for _ in range(T)]).astype(np.int32)
    x = synth.activations(T, VK, 93)
    xt = sc.f32(x.reshape(T, 1, VK))
    it = sc.i32(ids)
    y = sc.empty_f32((M, k, T))
    be.mul_mat_id(ev, xt, it, y)
    be.synchronize()
    got = be.get_f32(y).reshape(T, k, M)
    for t in range(T):
        for j in range(k):
            xb = raw[(3 + ids[t, j]) * mat:(4 + ids[t, j]) * mat]
            ref = orc.mul_mat(qtype, xb, M, VK, x[t:t + 1])
            assert rel_err(got[t, j][None], ref) <= TOL, (t, j)


# ------------------------------------------------------------------ bit-exact
@pytest.mark.parametrize("qtype", TYPES)
def test_dequant_bit_exact(be, sc, orc, qtype):
    say("dequant", qtype)
    blck, bb = synth.BLOCK[qtype]
    nblk = 4096 if blck == 32 else 1024
    raw = special_blocks(qtype, nblk, seed=31)
    n = nblk * blck
    w = sc.weights(qtype, raw, (n // 8, 8))
    y = sc.empty_f32((n // 8, 8))
    be.dequantize(w, y)
    be.synchronize()
    got = be.get_tensor(y).view(np.uint32)
    ref = orc.dequantize(qtype, raw, n).view(np.uint32)
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} of {n} values differ"


def act_cases(K, seed):
    g = np.random.default_rng(seed)
    x = g.standard_normal((6, K)).astype(np.float32)
    x[1, :] = 0.0                                      # all-zero blocks
    x[2, :] = np.round(x[2, :] * 4) / 4                # many exact ties after scaling
    x[2, 0:256:32] = 127.0 / 4
    x[3, :] = 1.0
    x[4, 5], x[4, 100] = -9.0, 9.0                     # equal |x|, opposite signs: first wins
    x[4, 300], x[4, 301] = 9.0, -9.0
    x[5, :] *= 1e-30                                   # tiny values
    return x


@pytest.mark.parametrize("act", [qmm.Q8_0, qmm.Q8_K])
def test_quantize_act_bit_exact(be, sc, orc, act):
    say("quantize_act", act)
    K = 1024
    x = act_cases(K, seed=41)
    xt = sc.f32(x)
    got = be.quantize_act(act, xt)
    ref = np.concatenate([orc.quantize_q8_0(r) if act == qmm.Q8_0 else orc.quantize_q8_K(r) for r in x])
    assert np.array_equal(got, ref)


def test_quantize_act_exact_ties(be, sc):
    """exact .5 ties under each quantizer's scale round half to even on the GPU: q8_K with a
    first max-|x| of -127 (iscale 1), q8_0 with amax 63.5 (multiplier 2, d = fp16 0.5)"""
    from test_oracle import q8k_tie_block
    say("quantize_act ties")
    x, want = q8k_tie_block()
    b = be.quantize_act(qmm.Q8_K, sc.f32(x[None, :]))
    assert b[0:4].view(np.float32)[0] == np.float32(1.0)
    assert np.array_equal(b[4:260].view(np.int8), want)
    # q8_0: values k / 2 + 1 / 4 scale by 2 to k + 1 / 2
    k = np.arange(31) - 15
    x0 = np.concatenate([[63.5], k / 2.0 + 0.25]).astype(np.float32)
    b0 = be.quantize_act(qmm.Q8_0, sc.f32(x0[None, :]))
    assert b0[0:2].view(np.float16)[0] == np.float16(0.5)
    assert np.array_equal(b0[2:34].view(np.int8), np.concatenate([[127], np.where(k % 2 == 0, k, k + 1)]).astype(np.int8))


def tiled_expected(orc, vdt, x, ntb):
    """The streaming GEMM's tiled activations from the oracle's quantization of x [N, K]: A
    [tile][32-weight block][lane half h][column i][16 codes], D [tile][scale block][32] f32 in
    MFMA output order (column i at 16 ((i >> 2) & 1) + 4 (i >> 3) + (i & 3)), and for q8_K S
    [tile][super-block][column][bh[8], bl[8]] with each sub-block sum = 64 bh + bl."""
    N, K = x.shape
    nblk = K // 32
    codes = np.zeros((ntb * 32, K), np.int8)
    if vdt == qmm.Q8_K:
        nsb = K // 256
        q = orc.quantize_q8_K(x).reshape(N, nsb, 292)
        d = np.zeros((ntb * 32, nsb), np.float32)
        d[:N] = q[:, :, 0:4].copy().view(np.float32)[:, :, 0]
        codes[:N] = q[:, :, 4:260].view(np.int8).reshape(N, K)
        bs = np.zeros((ntb * 32, nsb, 8), np.int64)
        bs[:N] = q[:, :, 260:292].copy().view(np.int16).reshape(N, nsb, 8, 2).sum(-1)
    else:
        nsb = nblk
        q = orc.quantize_q8_0(x).reshape(N, nblk, 34)
        d = np.zeros((ntb * 32, nblk), np.float32)
        d[:N] = q[:, :, 0:2].copy().view(np.float16)[:, :, 0].astype(np.float32)
        codes[:N] = q[:, :, 2:34].view(np.int8).reshape(N, K)
    A = codes.reshape(ntb, 32, nblk, 2, 16).transpose(0, 2, 3, 1, 4)
    pos = np.array([16 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3) for i in range(32)])
    D = np.zeros((ntb, nsb, 32), np.float32)
    D[:, :, pos] = d.reshape(ntb, 32, nsb).transpose(0, 2, 1)
    parts = [A.ravel().view(np.uint8), D.ravel().view(np.uint8)]
    if vdt == qmm.Q8_K:
        bsr = bs.reshape(ntb, 32, nsb, 8).transpose(0, 2, 1, 3)
        S = np.concatenate([bsr >> 6, bsr & 63], -1).astype(np.int8)
        parts.append(S.ravel().view(np.uint8))
    return np.concatenate(parts)


@pytest.mark.parametrize("qtype", [qmm.Q4_0, qmm.Q4_K])
@pytest.mark.parametrize("N,K", [(1, 256), (33, 512), (64, 2048), (100, 768)])
def test_quantize_tiled(be, sc, orc, qtype, N, K):
    """the streaming GEMM's tiled pre-pass is the oracle's quantization, laid out as the kernel
    reads it (columns past N zero)"""
    import ctypes as C
    say("quantize_tiled", qtype, N, K)
    x = synth.activations(N, K, seed=N + K)
    x[0, 7] = -3 * np.abs(x[0]).max()                          # a negative first maximum
    if N > 3:
        x[3, :] = 0.0                                          # an all-zero column
    ntb = -(-N // 32)
    want = tiled_expected(orc, qmm.Q8_K if qtype == qmm.Q4_K else qmm.Q8_0, x, ntb)
    L = qmm.load()
    f = L.qmm_internal_quantize_tiled
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int64]
    f.restype = C.c_int64
    out = np.zeros(want.size + 64, np.uint8)
    xt = sc.f32(x)
    n = f(be.h, C.byref(xt.c), qtype, out.ctypes.data, out.size)
    assert n == want.size
    got = out[:n]
    nA = ntb * (K // 32) * 1024
    assert np.array_equal(got[:nA], want[:nA]), "codes"
    nD = ntb * (K // (256 if qtype == qmm.Q4_K else 32)) * 128
    assert np.array_equal(got[nA:nA + nD], want[nA:nA + nD]), "scales"
    assert np.array_equal(got[nA + nD:], want[nA + nD:]), "split sums"


# ------------------------------------------------------------------ MUL_MAT
def run_mul_mat(be, sc, orc, qtype, M, K, N, seed):
    raw = synth.weights(qtype, M, K, seed)
    x = synth.activations(N, K, seed + 1)
    w = sc.weights(qtype, raw, (K, M))
    xt = sc.f32(x)
    y = sc.empty_f32((M, N))
    be.mul_mat(w, xt, y)
    be.synchronize()
    got = be.get_f32(y).reshape(N, M)
    ref = orc.mul_mat(qtype, raw, M, K, x)
    return got, ref


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("N", [1, 2, 3, 4, 5, 8])
def test_mul_mat_gemv(be, sc, orc, monkeypatch, qtype, N):
    """the pre-pass GEMV kernels (the fused one, which small 1-2 column products take by
    default, has its own tests)"""
    monkeypatch.setenv("QMM_GEMV_FQ_SMALL_TG", "0")
    monkeypatch.setenv("QMM_GEMV_FQS", "0")
    M, K = 300, 2048
    say("gemv", qtype, M, K, N)
    got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=51)
    # 3..8 columns of the types the MFMA kernel decodes run on it
    mma = N >= 3 and qtype in MMA_TYPES
    assert be.last_path() == ("gemv-mfma" if mma else "gemv")
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("K", [256, 512, 768, 5120])
def test_mul_mat_k_shapes(be, sc, orc, qtype, K):
    M, N = 129, 1
    say("gemv-k", qtype, M, K, N)
    got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=52)
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("qtype", [qmm.Q4_0, qmm.Q8_0, qmm.IQ4_NL])
@pytest.mark.parametrize("K", [640, 32 * 13])
@pytest.mark.parametrize("N", [1, 5, 20])
def test_mul_mat_k_not_whole_groups(be, sc, orc, qtype, K, N):
    """32-weight block types with K not a multiple of 256 (the reference's IQ4_NL down
    projections have K = 640, P01:3414-3416): the last group is zero-padded in the image"""
    M = 200
    say("k-partial", qtype, M, K, N)
    got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=53)
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("N", [9, 16, 37])
def test_mul_mat_many_columns(be, sc, orc, qtype, N):
    M, K = 96, 1024
    say("gemv-many", qtype, M, K, N)
    got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=53)
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("qtype", list(MMA_TYPES))
@pytest.mark.parametrize("N", [9, 12, 16, 17, 24, 31, 32, 40, 64, 100])
def test_mfma_gemv_wide_tasks(be, sc, orc, monkeypatch, qtype, N):
    """the MFMA GEMV with 9..32 columns per weight pass (the 16- and 32-column kernels; 40 and
    up in even passes), forced off the GEMM and off the fused kernel (which takes small products
    to 16 columns)"""
    monkeypatch.setenv("QMM_GEMM_MIN_COLS", "100000")
    monkeypatch.setenv("QMM_GEMV_FQ_SMALL_TG", "0")
    M, K = 300, 1024
    say("gemv-wide", qtype, M, K, N)
    got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=54)
    assert be.last_path() == "gemv-mfma"
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q4_0])
def test_mfma_gemv_wide_broadcast_and_strides(be, sc, orc, monkeypatch, qtype):
    monkeypatch.setenv("QMM_GEMM_MIN_COLS", "100000")
    monkeypatch.setenv("QMM_GEMV_FQ_SMALL_TG", "0")
    say("gemv-wide-broadcast", qtype)
    K, M, N = 512, 80, 21
    raw = synth.weights(qtype, 2 * M, K, seed=66)
    w = sc.weights(qtype, raw, (K, M, 2))
    x = synth.activations(4 * N, K, seed=67).reshape(4, N, K)
    ypad = sc.empty_f32((M + 5, N, 4))
    yv = qmm.Tensor(ypad.buf, qmm.F32, (M, N, 4), nb=(4, 4 * (M + 5), 4 * (M + 5) * N, 4 * (M + 5) * N * 4))
    be.mul_mat(w, sc.f32(x), yv)
    be.synchronize()
    assert be.last_path() == "gemv-mfma"
    got = be.get_f32(ypad).reshape(4, N, M + 5)[:, :, :M]
    rb = synth.row_bytes(qtype, K) * M
    for i2 in range(4):
        assert rel_err(got[i2], orc.mul_mat(qtype, raw[(i2 // 2) * rb:(i2 // 2 + 1) * rb], M, K, x[i2])) <= TOL


def test_mul_mat_broadcast_and_strides(be, sc, orc):
    say("broadcast")
    qtype, K, M, N = qmm.Q4_K, 512, 64, 3
    raw = synth.weights(qtype, 2 * M, K, seed=61)          # ne02 = 2 matrices
    w = sc.weights(qtype, raw, (K, M, 2))
    x = synth.activations(4 * N, K, seed=62).reshape(4, N, K)   # ne12 = 4 -> r2 = 2
    xt = sc.f32(x)
    y = sc.empty_f32((M, N, 4))
    be.mul_mat(w, xt, y)
    be.synchronize()
    got = be.get_f32(y).reshape(4, N, M)
    rb = synth.row_bytes(qtype, K) * M
    for i2 in range(4):
        ref = orc.mul_mat(qtype, raw[(i2 // 2) * rb:(i2 // 2 + 1) * rb], M, K, x[i2])
        assert rel_err(got[i2], ref) <= TOL
    # a strided src1 view (every other column) and a padded dst
    xs = synth.activations(2 * N, K, seed=63)
    xst = sc.f32(xs)
    w2 = sc.weights(qtype, raw[:rb], (K, M))
    view = qmm.Tensor(xst.buf, qmm.F32, (K, N), nb=(4, 8 * K, 8 * K * N, 8 * K * N))
    ypad = sc.empty_f32((M + 5, N))
    yview = qmm.Tensor(ypad.buf, qmm.F32, (M, N), nb=(4, 4 * (M + 5), 4 * (M + 5) * N, 4 * (M + 5) * N))
    be.mul_mat(w2, view, yview)
    be.synchronize()
    got = be.get_f32(ypad).reshape(N, M + 5)[:, :M]
    ref = orc.mul_mat(qtype, raw[:rb], M, K, xs[0::2])
    assert rel_err(got, ref) <= TOL


# ------------------------------------------------------------------ MUL_MAT_ID
@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("T", [1, 4, 19])
@pytest.mark.parametrize("bcast", [True, False])
def test_mul_mat_id(be, sc, orc, qtype, T, bcast):
    E, n_used, M = 16, 4, 96
    K = 512
    say("mul_mat_id", qtype, T, bcast)
    raw = synth.weights(qtype, E * M, K, seed=71)
    ids = synth.moe_ids(T, E, n_used, seed=72)
    if T >= 4:
        ids[1, 2] = -1                                   # a negative id writes zeros
    ne11 = 1 if bcast else n_used
    x = synth.activations(T * ne11, K, seed=73).reshape(T, ne11, K)
    w = sc.weights(qtype, raw, (K, M, E))
    xt = sc.f32(x)
    it = sc.i32(ids)
    y = sc.empty_f32((M, n_used, T))
    be.mul_mat_id(w, xt, it, y)
    be.synchronize()
    got = be.get_f32(y).reshape(T, n_used, M)
    ref = orc.mul_mat_id(qtype, raw, M, K, E, x, ids)
    assert rel_err(got, ref) <= TOL
    if T >= 4:
        assert not got[1, 2].any()


@pytest.mark.parametrize("T", [1024, 1100])
def test_mul_mat_id_many_pairs(be, sc, orc, T):
    """4096 and 4400 (token, slot) pairs: a route over several pairs per route thread, about
    275 pairs per expert in tasks of 8, one invalid id"""
    qtype, E, n_used, M, K = qmm.Q4_K, 16, 4, 64, 256
    say("mul_mat_id many pairs", T)
    raw = synth.weights(qtype, E * M, K, seed=77)
    ids = synth.moe_ids(T, E, n_used, seed=78)
    ids[T - 1, 3] = -1
    x = synth.activations(T, K, seed=79).reshape(T, 1, K)
    w = sc.weights(qtype, raw, (K, M, E))
    y = sc.empty_f32((M, n_used, T))
    be.mul_mat_id(w, sc.f32(x), sc.i32(ids), y)
    be.synchronize()
    got = be.get_f32(y).reshape(T, n_used, M)
    assert rel_err(got, orc.mul_mat_id(qtype, raw, M, K, E, x, ids)) <= TOL
    assert not got[T - 1, 3].any()


GROUPED_TYPES = [qmm.Q4_K, qmm.Q6_K, qmm.Q5_K, qmm.IQ4_XS]


@pytest.mark.parametrize("qtype", GROUPED_TYPES)
@pytest.mark.parametrize("bcast,K", [(True, 1280), (False, 1280), (False, 512)])
def test_mul_mat_id_grouped_gemm(be, sc, orc, monkeypatch, qtype, bcast, K):
    """MUL_MAT_ID on the grouped GEMM (experts averaging >= 32 pairs) of each type that has one:
    64-column units of one expert, activations gathered from the route's quantization; ragged:
    100 rows, 3 of 8 experts without pairs, pair counts not a multiple of 64, negative ids
    (zero rows); K = 512 (two super-blocks, the down shape) is the smallest K it takes"""
    E, n_used, M, T = 8, 3, 100, 300
    say("mul_mat_id grouped gemm", qtype, bcast, K)
    raw = synth.weights(qtype, E * M, K, seed=81)
    g = np.random.default_rng(82)
    ids = np.stack([g.choice([0, 2, 4, 5, 6], size=n_used, replace=False) for _ in range(T)]).astype(np.int32)
    ids[7, 1] = -1
    ids[11, 0] = -1
    ne11 = 1 if bcast else n_used
    x = synth.activations(T * ne11, K, seed=83).reshape(T, ne11, K)
    w = sc.weights(qtype, raw, (K, M, E))
    y = sc.empty_f32((M, n_used, T))
    be.mul_mat_id(w, sc.f32(x), sc.i32(ids), y)
    be.synchronize()
    assert be.last_path() == "gemm-id-stream"
    got = be.get_f32(y).reshape(T, n_used, M)
    assert rel_err(got, orc.mul_mat_id(qtype, raw, M, K, E, x, ids)) <= TOL
    assert not got[7, 1].any() and not got[11, 0].any()
    # the same op on the GEMV tasks agrees
    monkeypatch.setenv("QMM_MOE_GEMM_MIN", "0")
    y2 = sc.empty_f32((M, n_used, T))
    be.mul_mat_id(w, sc.f32(x), sc.i32(ids), y2)
    be.synchronize()
    assert be.last_path() != "gemm-id-stream"
    assert rel_err(got, be.get_f32(y2).reshape(T, n_used, M)) <= TOL


@pytest.mark.parametrize("qtype", GROUPED_TYPES)
@pytest.mark.parametrize("M,K,ne11,T", [(512, 2048, 1, 1024), (2048, 512, 10, 256)])
def test_mul_mat_id_grouped_gemm_config3_shape(be, sc, orc, qtype, M, K, ne11, T):
    """config 3's expert shapes with 16 experts, top-10, on the grouped GEMM's one-slice form
    (4-wave blocks, one K slice: mostly full units, a block per CU or more): gate/up 512 x 2048
    at 1024 tokens (ne11 = 1, 640 pairs per expert) and down 2048 x 512 at 256 (ne11 = 10, 160
    pairs per expert, K = 512)"""
    E, n_used = 16, 10
    say("mul_mat_id grouped gemm config3 shape", qtype, M, K, T)
    raw = synth.weights(qtype, E * M, K, seed=84)
    ids = synth.moe_ids(T, E, n_used, seed=85)
    x = synth.activations(T * ne11, K, seed=86).reshape(T, ne11, K)
    w = sc.weights(qtype, raw, (K, M, E))
    y = sc.empty_f32((M, n_used, T))
    be.mul_mat_id(w, sc.f32(x), sc.i32(ids), y)
    be.synchronize()
    assert be.last_path() == "gemm-id-stream"
    got = be.get_f32(y).reshape(T, n_used, M)
    assert rel_err(got, orc.mul_mat_id(qtype, raw, M, K, E, x, ids)) <= TOL


def test_mul_mat_id_glu_grouped_gemm_one_slice(be, sc, orc):
    """gate + up + SwiGLU on the grouped GEMM's one-slice form (16 experts of 512 x 2048 at 1024
    tokens, top-10): the gate launch, then the up launch applying the GLU at its stores"""
    from oracle import glu as G
    qtype, E, n_used, M, K, T = qmm.Q6_K, 16, 10, 512, 2048, 1024
    say("mul_mat_id_glu grouped gemm one slice", qtype)
    rg, ru = synth.weights(qtype, E * M, K, seed=87), synth.weights(qtype, E * M, K, seed=88)
    ids = synth.moe_ids(T, E, n_used, seed=89)
    x = synth.activations(T, K, seed=90).reshape(T, 1, K)
    wg, wu = sc.weights(qtype, rg, (K, M, E)), sc.weights(qtype, ru, (K, M, E))
    y = sc.empty_f32((M, n_used, T))
    be.mul_mat_id_glu(wg, wu, sc.f32(x), sc.i32(ids), y, qmm.GLU_SWIGLU)
    be.synchronize()
    assert be.last_path() == "glu-gemm-id-stream"
    got = be.get_f32(y).reshape(T, n_used, M)
    ref = G.glu(qmm.GLU_SWIGLU, orc.mul_mat_id(qtype, rg, M, K, E, x, ids), orc.mul_mat_id(qtype, ru, M, K, E, x, ids))
    assert rel_err(got, ref) <= TOL


def test_mul_mat_id_all_tokens_one_expert(be, sc, orc):
    # more than 8 pairs on one expert: several tasks per expert
    qtype, E, n_used, M, K, T = qmm.Q4_K, 4, 2, 64, 256, 40
    say("mul_mat_id-hot")
    raw = synth.weights(qtype, E * M, K, seed=74)
    ids = np.tile(np.array([[3, 1]], np.int32), (T, 1))
    x = synth.activations(T, K, seed=75).reshape(T, 1, K)
    w = sc.weights(qtype, raw, (K, M, E))
    y = sc.empty_f32((M, n_used, T))
    be.mul_mat_id(w, sc.f32(x), sc.i32(ids), y)
    be.synchronize()
    got = be.get_f32(y).reshape(T, n_used, M)
    assert rel_err(got, orc.mul_mat_id(qtype, raw, M, K, E, x, ids)) <= TOL


# ------------------------------------------------------------------ graph
def test_graph_activation_dedup(be, sc, orc):
    say("graph")
    K, M, N = 1024, 80, 2
    ra = synth.weights(qmm.Q4_K, M, K, seed=81)
    rb = synth.weights(qmm.Q6_K, M, K, seed=82)
    rc = synth.weights(qmm.Q4_0, M, K, seed=83)
    x = synth.activations(N, K, seed=84)
    wa, wb, wc = sc.weights(qmm.Q4_K, ra, (K, M)), sc.weights(qmm.Q6_K, rb, (K, M)), sc.weights(qmm.Q4_0, rc, (K, M))
    xt = sc.f32(x)
    ya, yb, yc = sc.empty_f32((M, N)), sc.empty_f32((M, N)), sc.empty_f32((M, N))
    be.graph_compute([(qmm.OP_MUL_MAT, wa, xt, None, ya), (qmm.OP_MUL_MAT, wb, xt, None, yb),
                      (qmm.OP_MUL_MAT, wc, xt, None, yc)])
    be.synchronize()
    assert rel_err(be.get_f32(ya).reshape(N, M), orc.mul_mat(qmm.Q4_K, ra, M, K, x)) <= TOL
    assert rel_err(be.get_f32(yb).reshape(N, M), orc.mul_mat(qmm.Q6_K, rb, M, K, x)) <= TOL
    assert rel_err(be.get_f32(yc).reshape(N, M), orc.mul_mat(qmm.Q4_0, rc, M, K, x)) <= TOL


# ------------------------------------------------------------------ full sizes
FULL = [
    (qmm.Q4_0, 4096, 4096), (qmm.Q4_0, 11008, 4096), (qmm.Q4_0, 4096, 11008),
    (qmm.Q4_K, 17408, 5120), (qmm.Q6_K, 5120, 17408), (qmm.Q4_K, 12288, 5120),
    (qmm.IQ4_XS, 14336, 4096), (qmm.IQ4_XS, 4096, 14336), (qmm.Q8_0, 14336, 4096), (qmm.Q8_0, 4096, 14336),
    (qmm.Q5_K, 17408, 5120), (qmm.Q5_K, 5120, 17408), (qmm.IQ4_NL, 14336, 4096), (qmm.IQ4_NL, 4096, 14336),
]


@pytest.mark.parametrize("qtype,M,K", FULL)
@pytest.mark.parametrize("N", [1, 4, 8])
def test_full_size_gemv(be, sc, orc, qtype, M, K, N):
    say("full", qtype, M, K, N)
    got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=91)
    assert rel_err(got, ref) <= TOL


# ------------------------------------------------------------------ MFMA GEMM (N >= 16)
@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("M,K,N", [(300, 1024, 16), (129, 2048, 37), (64, 512, 64), (500, 768, 130),
                                   (200, 256, 40), (70, 800, 20), (1000, 512, 300)])
def test_mul_mat_gemm(be, sc, orc, monkeypatch, qtype, M, K, N):
    monkeypatch.setenv("QMM_GEMM_MIN_COLS", "16")                 # the GEMM from 16 columns, every type
    if K % 256 and qtype not in (qmm.Q4_0, qmm.Q8_0, qmm.IQ4_NL):
        K = 1024
    say("gemm", qtype, M, K, N)
    got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=57)
    assert be.last_path() == gemm_path(qtype)
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("qtype", [qmm.Q6_K, qmm.Q4_K, qmm.Q5_K, qmm.Q4_0, qmm.IQ4_NL])
def test_mul_mat_gemm_broadcast_and_strides(be, sc, orc, monkeypatch, qtype):
    monkeypatch.setenv("QMM_GEMM_MIN_COLS", "16")
    say("gemm-broadcast", qtype)
    K, M, N = 512, 80, 21
    raw = synth.weights(qtype, 2 * M, K, seed=64)
    w = sc.weights(qtype, raw, (K, M, 2))
    x = synth.activations(4 * N, K, seed=65).reshape(4, N, K)
    y = sc.empty_f32((M, N, 4))
    be.mul_mat(w, sc.f32(x), y)
    be.synchronize()
    assert be.last_path() == gemm_path(qtype)
    got = be.get_f32(y).reshape(4, N, M)
    rb = synth.row_bytes(qtype, K) * M
    for i2 in range(4):
        ref = orc.mul_mat(qtype, raw[(i2 // 2) * rb:(i2 // 2 + 1) * rb], M, K, x[i2])
        assert rel_err(got[i2], ref) <= TOL
    ypad = sc.empty_f32((M + 3, N))
    yview = qmm.Tensor(ypad.buf, qmm.F32, (M, N), nb=(4, 4 * (M + 3), 4 * (M + 3) * N, 4 * (M + 3) * N))
    w2 = sc.weights(qtype, raw[:rb], (K, M))
    be.mul_mat(w2, sc.f32(x[1]), yview)
    be.synchronize()
    got = be.get_f32(ypad).reshape(N, M + 3)[:, :M]
    assert rel_err(got, orc.mul_mat(qtype, raw[:rb], M, K, x[1])) <= TOL


GEMM_FULL = [
    (qmm.Q4_0, 4096, 4096, 512), (qmm.Q4_0, 11008, 4096, 64), (qmm.Q4_0, 4096, 11008, 64),
    (qmm.Q4_K, 17408, 5120, 64), (qmm.Q6_K, 5120, 17408, 64), (qmm.IQ4_XS, 4096, 14336, 32),
    (qmm.Q8_0, 14336, 4096, 32), (qmm.Q5_K, 17408, 5120, 64), (qmm.IQ4_NL, 4096, 14336, 32),
]


@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q6_K])
def test_gemm_tail_split(be, sc, orc, monkeypatch, qtype):
    # 66 row tiles x 4 column tiles = 264 > 256 work-groups: the first 256 tiles run whole and
    # the last row of tiles (partial: 8384 = 65.5 x 128 rows) in K slices added into dst rows
    # the pre-pass zeroed (Q4_K and Q6_K on this kernel when the streaming ones are switched off)
    monkeypatch.setenv("QMM_GEMM3_Q4K", "0")
    monkeypatch.setenv("QMM_GEMM3_Q6K", "0")
    M, K, N = 8384, 1024, 512
    fake = qmm.Buffer(ptr=0x1000, size=1 << 44)
    info = qmm.describe_mul_mat(qmm.Tensor(fake, qtype, (K, M)), qmm.Tensor(fake, qmm.F32, (K, N)),
                                qmm.Tensor(fake, qmm.F32, (M, N)))
    assert info["path"] == "gemm-mfma" and info["k_slices"] > 1
    assert info["workgroups"] == 256 + 8 * info["k_slices"]
    say("gemm-tail", qtype, M, K, N)
    got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=95)
    assert be.last_path() == "gemm-mfma"
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("qtype,M,K,N", GEMM_FULL)
def test_full_size_gemm(be, sc, orc, monkeypatch, qtype, M, K, N):
    monkeypatch.setenv("QMM_GEMM_MIN_COLS", "16")
    say("gemm-full", qtype, M, K, N)
    got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=93)
    assert be.last_path() == gemm_path(qtype)
    assert rel_err(got, ref) <= TOL


# streaming GEMM of the block types: each launch shape (row-half waves U x K slices KS, forced
# by index) on ragged shapes (N not a multiple of 32 or of a column pair, a work-group's last
# row halves missing, K not a multiple of 256, K slices of unequal length: G = 17 over 3 or 4
# slices), batches with broadcast weights
@pytest.mark.parametrize("qtype", [qmm.Q4_0, qmm.Q8_0, qmm.IQ4_NL])
@pytest.mark.parametrize("KS", range(6))
def test_gemm_stream_shapes(be, sc, orc, monkeypatch, qtype, KS):
    monkeypatch.setenv("QMM_GEMM3_KQ", str(KS))
    monkeypatch.setenv("QMM_GEMM_MIN_COLS", "16")                 # (small shapes: the GEMM regardless)
    for (M, K, N, seed) in [(200, 800, 33, 301), (64, 2048, 100, 302), (130, 512, 64, 303), (448, 1280, 161, 304),
                            (700, 4352, 40, 307)]:
        say("gemm-stream", qtype, KS, M, K, N)
        got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=seed)
        assert be.last_path() == "gemm-stream"
        assert rel_err(got, ref) <= TOL, (M, K, N)
    say("gemm-stream batches", qtype, KS)
    K, M, N = 768, 96, 45
    raw = synth.weights(qtype, 2 * M, K, seed=305)
    w = sc.weights(qtype, raw, (K, M, 2))
    x = synth.activations(4 * N, K, seed=306).reshape(4, N, K)
    y = sc.empty_f32((M, N, 4))
    be.mul_mat(w, sc.f32(x), y)
    be.synchronize()
    assert be.last_path() == "gemm-stream"
    got = be.get_f32(y).reshape(4, N, M)
    rb = synth.row_bytes(qtype, K) * M
    for i2 in range(4):
        ref = orc.mul_mat(qtype, raw[(i2 // 2) * rb:(i2 // 2 + 1) * rb], M, K, x[i2])
        assert rel_err(got[i2], ref) <= TOL


# the tail blocks of a one-slice launch in K pieces that meet in tree slots: 2, 3 and 4
# pieces (G = 4, 5 and 17 over the forced 4-wave shape, whose 768 slots the few blocks leave
# mostly empty), against the oracle, the same bits on a second call (every slot is left empty,
# and a + b = b + a whichever piece arrives first) and within rounding of whole blocks
# (QMM_GEMM3_TAIL=0)
@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q4_0, qmm.IQ4_NL])
def test_gemm_tail_pieces(be, sc, orc, monkeypatch, qtype):
    monkeypatch.setenv("QMM_GEMM3_KQ", "4")
    monkeypatch.setenv("QMM_GEMM_MIN_COLS", "16")
    fake = qmm.Buffer(ptr=0x1000, size=1 << 44)
    for (M, K, N, ts, seed) in [(200, 1024, 33, 2, 321), (448, 1280, 161, 3, 322), (700, 4352, 40, 4, 323)]:
        say("gemm-tail", qtype, M, K, N, ts)
        info = qmm.describe_mul_mat(qmm.Tensor(fake, qtype, (K, M)), qmm.Tensor(fake, qmm.F32, (K, N)),
                                    qmm.Tensor(fake, qmm.F32, (M, N)))
        nwg = -(-(2 * -(-M // 64)) // 4) * -(-(-(-N // 32)) // 2)
        assert info["workgroups"] == 8 * -(-(nwg * ts) // 8), (info, nwg, ts)
        got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=seed)
        assert be.last_path() == "gemm-stream"
        assert rel_err(got, ref) <= TOL, (M, K, N)
        again, _ = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=seed)
        assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
        monkeypatch.setenv("QMM_GEMM3_TAIL", "0")
        whole, _ = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=seed)
        monkeypatch.delenv("QMM_GEMM3_TAIL")
        assert rel_err(got, whole) <= 1e-4                       # (the same float sums in another order)


# Q4_K streaming GEMM: each launch shape (row-half waves U x K slices KS, forced by index) on
# ragged shapes: rows not a whole number of 32-row halves or of a work-group's U, column tiles
# not a whole number of pairs (N = 80: 3 tiles), K slices of unequal length (G = 17 over 3 or
# 4 slices), a single super-block, batches with broadcast weights
@pytest.mark.parametrize("shape", range(6))
def test_gemm_stream_q4k_shapes(be, sc, orc, monkeypatch, shape):
    monkeypatch.setenv("QMM_GEMM3_KQ", str(shape))
    monkeypatch.setenv("QMM_GEMM_MIN_COLS", "16")
    qtype = qmm.Q4_K
    for (M, K, N, seed) in [(200, 768, 33, 311), (64, 2048, 100, 312), (130, 256, 64, 313), (448, 1280, 161, 314),
                            (330, 4352, 80, 317), (1000, 1024, 128, 318)]:
        say("gemm-stream q4k", shape, M, K, N)
        got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=seed)
        assert be.last_path() == "gemm-stream"
        assert rel_err(got, ref) <= TOL, (M, K, N)
    say("gemm-stream q4k batches", shape)
    K, M, N = 512, 96, 45
    raw = synth.weights(qtype, 2 * M, K, seed=315)
    w = sc.weights(qtype, raw, (K, M, 2))
    x = synth.activations(4 * N, K, seed=316).reshape(4, N, K)
    y = sc.empty_f32((M, N, 4))
    be.mul_mat(w, sc.f32(x), y)
    be.synchronize()
    assert be.last_path() == "gemm-stream"
    got = be.get_f32(y).reshape(4, N, M)
    rb = synth.row_bytes(qtype, K) * M
    for i2 in range(4):
        ref = orc.mul_mat(qtype, raw[(i2 // 2) * rb:(i2 // 2 + 1) * rb], M, K, x[i2])
        assert rel_err(got[i2], ref) <= TOL


# ------------------------------------------------------------------ MoE router and combine
@pytest.mark.parametrize("n_expert,k", [(8, 2), (64, 8), (100, 10), (512, 10), (1024, 32), (32, 32)])
@pytest.mark.parametrize("T", [1, 5, 37])
def test_moe_topk(be, sc, orc, n_expert, k, T):
    from oracle import moe
    say("moe_topk", n_expert, k, T)
    g = np.random.default_rng(n_expert * 7 + k * 3 + T)
    logits = (g.standard_normal((T, n_expert)) * 3).astype(np.float32)
    logits[0, : n_expert // 2] = logits[0, 0]                # one token with a run of equal logits
    lt = sc.f32(logits)
    ids = sc.i32(np.zeros((T, k), np.int32))
    w = sc.empty_f32((k, T))
    be.moe_topk(lt, ids, w)
    be.synchronize()
    got_ids = be.get_tensor(ids).view(np.int32).reshape(T, k)
    got_w = be.get_f32(w).reshape(T, k)
    ref_ids, ref_w = moe.topk(logits, k, 6.103515625e-5, np.inf)
    assert np.array_equal(got_ids, ref_ids)
    np.testing.assert_allclose(got_w, ref_w, rtol=2e-6, atol=1e-30)


def test_moe_topk_float32_exp_ties(be, sc, orc):
    """the router ranks the float32 values exp(x - max): logits -1e-8 and -2e-8 (experts 5 and 7)
    have the maximum's exp, 1.0f, so the three tie and go in expert order, ahead of the maximum
    (expert 300); logit order would put 300 first (the oracle's own case, test_oracle_moe.py)"""
    from oracle import moe
    say("moe_topk float32 exp ties")
    logits = np.full((2, 400), -3.0, np.float32)
    logits[:, 300] = 0.0
    logits[:, 7] = -2e-8
    logits[:, 5] = -1e-8
    logits[:, 9] = -0.5
    ids = sc.i32(np.zeros((2, 4), np.int32))
    w = sc.empty_f32((4, 2))
    be.moe_topk(sc.f32(logits), ids, w, 0.0, float("inf"))
    be.synchronize()
    got_ids = be.get_tensor(ids).view(np.int32).reshape(2, 4)
    ref_ids, ref_w = moe.topk(logits, 4, 0.0, np.inf)
    assert [list(r) for r in ref_ids] == [[5, 7, 300, 9]] * 2
    assert np.array_equal(got_ids, ref_ids)
    np.testing.assert_allclose(be.get_f32(w).reshape(2, 4), ref_w, rtol=2e-6)


def test_moe_topk_clamp_and_views(be, sc, orc):
    from oracle import moe
    say("moe_topk_clamp")
    T, n_expert, k = 6, 96, 4
    g = np.random.default_rng(77)
    logits = (g.standard_normal((T, n_expert)) * 5).astype(np.float32)
    # logits as a view with padded rows, ids / weights into wider rows
    pad = np.zeros((T, n_expert + 7), np.float32)
    pad[:, :n_expert] = logits
    lp = sc.f32(pad)
    lv = qmm.Tensor(lp.buf, qmm.F32, (n_expert, T), nb=(4, 4 * (n_expert + 7), 4 * (n_expert + 7) * T,
                                                           4 * (n_expert + 7) * T))
    ib = sc.i32(np.zeros((T, k + 3), np.int32))
    iv = qmm.Tensor(ib.buf, qmm.I32, (k, T), nb=(4, 4 * (k + 3), 4 * (k + 3) * T, 4 * (k + 3) * T))
    wb = sc.empty_f32((k + 3, T))
    wv = qmm.Tensor(wb.buf, qmm.F32, (k, T), nb=(4, 4 * (k + 3), 4 * (k + 3) * T, 4 * (k + 3) * T))
    be.moe_topk(lv, iv, wv, 0.0, 0.5)
    be.synchronize()
    got_ids = be.get_tensor(ib).view(np.int32).reshape(T, k + 3)[:, :k]
    got_w = be.get_f32(wb).reshape(T, k + 3)[:, :k]
    ref_ids, ref_w = moe.topk(logits, k, 0.0, 0.5)
    assert np.array_equal(got_ids, ref_ids)
    np.testing.assert_allclose(got_w, ref_w, rtol=2e-6)
    with pytest.raises(qmm.QmmError):                          # k above 32
        be.moe_topk(sc.f32(logits), sc.i32(np.zeros((T, 33), np.int32)), sc.empty_f32((33, T)))


@pytest.mark.parametrize("shared", [False, True])
def test_moe_combine(be, sc, orc, shared):
    from oracle import moe
    say("moe_combine", shared)
    T, k, M = 7, 10, 333
    g = np.random.default_rng(11 + shared)
    e = g.standard_normal((T, k, M)).astype(np.float32)
    w = g.random((T, k)).astype(np.float32)
    s = g.standard_normal((T, M)).astype(np.float32) if shared else None
    gt = g.standard_normal(T).astype(np.float32) * 2 if shared else None
    y = sc.empty_f32((M, T))
    be.moe_combine(sc.f32(e), sc.f32(w), y, sc.f32(s) if shared else None,
                   sc.f32(gt.reshape(T, 1)) if shared else None)
    be.synchronize()
    got = be.get_f32(y).reshape(T, M)
    ref = moe.combine(e, w, s, gt)
    if shared:                                                 # the sigmoid's expf may differ by an ulp
        np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)
    else:                                                      # same products and order: bit-exact
        assert np.array_equal(got, ref)


def test_moe_layer_end_to_end(be, sc, orc):
    """router -> MUL_MAT_ID (gate/up style, one activation column per token) -> combine,
    against the oracle's router, per-expert products and combine"""
    from oracle import moe
    say("moe_layer")
    E, k, T, K, M = 16, 4, 5, 512, 96
    g = np.random.default_rng(123)
    logits = (g.standard_normal((T, E)) * 2).astype(np.float32)
    raw = synth.weights(qmm.Q4_K, E * M, K, seed=124)
    x = synth.activations(T, K, seed=125)
    w = sc.weights(qmm.Q4_K, raw, (K, M, E))
    ids = sc.i32(np.zeros((T, k), np.int32))
    wts = sc.empty_f32((k, T))
    be.moe_topk(sc.f32(logits), ids, wts)
    xt = sc.f32(x.reshape(T, 1, K))
    ex = sc.empty_f32((M, k, T))
    be.mul_mat_id(w, xt, ids, ex)
    y = sc.empty_f32((M, T))
    be.moe_combine(ex, wts, y)
    be.synchronize()
    got = be.get_f32(y).reshape(T, M)
    ref_ids, ref_w = moe.topk(logits, k, 6.103515625e-5, np.inf)
    rb = synth.row_bytes(qmm.Q4_K, K) * M
    ref_e = np.zeros((T, k, M), np.float32)
    for t in range(T):
        for j in range(k):
            e = int(ref_ids[t, j])
            ref_e[t, j] = orc.mul_mat(qmm.Q4_K, raw[e * rb:(e + 1) * rb], M, K, x[t:t + 1])[0]
    ref = moe.combine(ref_e, ref_w.astype(np.float32))
    assert rel_err(got, ref) <= TOL


# ------------------------------------------------------------------ gate/up + GLU
GLU_OPS = [qmm.GLU_REGLU, qmm.GLU_GEGLU, qmm.GLU_SWIGLU, qmm.GLU_GEGLU_ERF, qmm.GLU_GEGLU_QUICK]


def glu_case(be, sc, orc, gtype, utype, M, K, N, op, seed, batches=(1, 1)):
    from oracle import glu as G
    b2, b3 = batches
    rg, ru = synth.weights(gtype, M, K, seed), synth.weights(utype, M, K, seed + 1)
    wg, wu = sc.weights(gtype, rg, (K, M)), sc.weights(utype, ru, (K, M))
    x = synth.activations(N * b2 * b3, K, seed + 2)
    xt = sc.f32(x.reshape(b3, b2, N, K))
    y = sc.empty_f32((M, N, b2, b3))
    be.mul_mat_glu(wg, wu, xt, y, op)
    be.synchronize()
    got = be.get_f32(y).reshape(b2 * b3 * N, M)
    ref = G.glu(op, orc.mul_mat(gtype, rg, M, K, x), orc.mul_mat(utype, ru, M, K, x))
    return got, ref


@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q4_0, qmm.Q6_K, qmm.Q5_K, qmm.IQ4_NL])
@pytest.mark.parametrize("N", [1, 4, 20])
def test_mul_mat_glu_fused(be, sc, orc, qtype, N):
    """one GEMV launch over gate and up (both images, the same columns), then the GLU"""
    M, K = 300, 1024
    if N >= 16 and qtype == qmm.Q5_K:
        N = 12                                                        # its GEMM starts at 16
    say("glu-fused", qtype, N)
    got, ref = glu_case(be, sc, orc, qtype, qtype, M, K, N, qmm.GLU_SWIGLU, seed=101)
    assert be.last_path().startswith("glu-fused-gemv")
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("op", GLU_OPS)
def test_mul_mat_glu_ops(be, sc, orc, op):
    say("glu-op", op)
    got, ref = glu_case(be, sc, orc, qmm.Q4_K, qmm.Q4_K, 256, 512, 2, op, seed=111)
    assert rel_err(got, ref) <= TOL


def test_mul_mat_glu_split_paths(be, sc, orc, monkeypatch):
    """the unfused forms: mixed weight types, the GEMM (forced on this small shape), broadcast
    batches"""
    say("glu-split mixed")
    got, ref = glu_case(be, sc, orc, qmm.Q4_K, qmm.Q6_K, 200, 1024, 3, qmm.GLU_SWIGLU, seed=121)
    assert be.last_path().startswith("glu-") and not be.last_path().startswith("glu-fused")
    assert rel_err(got, ref) <= TOL
    say("glu-split gemm")
    with monkeypatch.context() as mp:
        mp.setenv("QMM_GEMM_MIN_COLS", "33")
        got, ref = glu_case(be, sc, orc, qmm.Q4_0, qmm.Q4_0, 200, 1024, 40, qmm.GLU_GEGLU, seed=122)
        assert be.last_path() == "glu-gemm-stream"
    assert rel_err(got, ref) <= TOL
    say("glu-split batches")
    got, ref = glu_case(be, sc, orc, qmm.Q4_K, qmm.Q4_K, 130, 512, 2, qmm.GLU_SWIGLU, seed=123, batches=(3, 2))
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q4_0, qmm.Q6_K, qmm.IQ4_XS, qmm.Q8_0])
@pytest.mark.parametrize("N,W", [(1, 4), (2, 3), (1, 1)])
def test_mul_mat_glu_split_tree(be, sc, orc, monkeypatch, qtype, N, W):
    """gate/up + GLU in one launch with K split over work-groups: each slice streams its gate and
    up groups, the slices' (gate, up) pairs meet in the exchange tree as one 64-bit exchange and
    the last arrival applies the GLU (K = 5120: 20 groups, slices of 4, 3 and 1 groups); two
    calls in a row on one context (the slots empty again after each)"""
    monkeypatch.setenv("QMM_GEMV_FQS", "1")
    monkeypatch.setenv("QMM_GEMV_FQS_W", str(W))
    monkeypatch.setenv("QMM_GEMV_FQ_SMALL_TG", "0")
    for seed in (141, 151):
        say("glu split tree", qtype, N, W, seed)
        got, ref = glu_case(be, sc, orc, qtype, qtype, 130, 5120, N, qmm.GLU_SWIGLU, seed=seed)
        assert be.last_path() == "glu-fused-gemv-fq"
        assert rel_err(got, ref) <= TOL, seed


@pytest.mark.parametrize("op", GLU_OPS)
def test_mul_mat_glu_split_tree_ops_batches(be, sc, orc, monkeypatch, op):
    """every GLU applied at the tree's root, over broadcast batches"""
    monkeypatch.setenv("QMM_GEMV_FQS", "1")
    monkeypatch.setenv("QMM_GEMV_FQS_W", "2")
    monkeypatch.setenv("QMM_GEMV_FQ_SMALL_TG", "0")
    say("glu split tree op", op)
    got, ref = glu_case(be, sc, orc, qmm.Q4_K, qmm.Q4_K, 200, 1536, 2, op, seed=161, batches=(3, 2))
    assert be.last_path() == "glu-fused-gemv-fq"
    assert rel_err(got, ref) <= TOL


def test_mul_mat_glu_full_size_decode(be, sc, orc):
    """config 2's FFN gate/up (17408 x 5120 Q4_K) at N = 1"""
    say("glu-full")
    got, ref = glu_case(be, sc, orc, qmm.Q4_K, qmm.Q4_K, 17408, 5120, 1, qmm.GLU_SWIGLU, seed=131)
    assert be.last_path().startswith("glu-fused-gemv")
    assert rel_err(got, ref) <= TOL


def test_mul_mat_glu_rejects(be, sc):
    K, M = 512, 64
    w1 = sc.weights(qmm.Q4_K, synth.weights(qmm.Q4_K, M, K, 1), (K, M))
    w2 = sc.weights(qmm.Q4_K, synth.weights(qmm.Q4_K, 2 * M, K, 2), (K, 2 * M))
    x, y = sc.f32(synth.activations(1, K, 3)), sc.empty_f32((M, 1))
    with pytest.raises(qmm.QmmError):
        be.mul_mat_glu(w1, w2, x, y, qmm.GLU_SWIGLU)                 # shapes differ
    with pytest.raises(qmm.QmmError):
        be.mul_mat_glu(w1, w1, x, y, 3)                              # SWIGLU_OAI is not taken


# ------------------------------------------------------------------ permuted src1
@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("nr", [4, 8, 12])
def test_mul_mat_permuted_src1(be, sc, orc, qtype, nr):
    """test-backend-ops' permuted src1 (the reference's review cases m = 256, n = 1, k = 2048,
    nr = 4 / 8 / 12, per = [0, 2, 1, 3], contrib/llama.cpp/README.md:6864): src1 [K, 1, nr] is a
    permutation of a contiguous [K, nr, 1], so nb1 = 4 K nr and nb2 = 4 K; the activation prep
    must step columns by the strides, not by 4 K"""
    M, K = 256, 2048
    say("permuted-src1", qtype, nr)
    raw = synth.weights(qtype, M, K, seed=141)
    w = sc.weights(qtype, raw, (K, M))
    x = synth.activations(nr, K, seed=142)                      # row i2: the activation of batch i2
    base = sc.f32(x)                                            # contiguous [K, nr]
    xp = qmm.Tensor(base.buf, qmm.F32, (K, 1, nr), nb=(4, 4 * K * nr, 4 * K, 4 * K * nr))
    y = sc.empty_f32((M, 1, nr))
    be.mul_mat(w, xp, y)
    be.synchronize()
    got = be.get_f32(y).reshape(nr, M)
    assert rel_err(got, orc.mul_mat(qtype, raw, M, K, x)) <= TOL


# ------------------------------------------------------------------ MoE: invalid ids, the route cache
@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q4_0])
@pytest.mark.parametrize("T", [1, 6, 40])
def test_mul_mat_id_invalid_ids_write_zero_rows(be, sc, orc, qtype, T):
    """negative ids (the reference's rule, P02:98-103) write zero rows over whatever dst held, on
    the v_dot4 and (T = 40: 160 pairs on 16 experts) MFMA task paths; ids at or past the expert
    count, which ggml-cpu asserts on (P02:105), write zero rows too and make the next
    synchronize report the error (once)"""
    E, n_used, M, K = 16, 4, 130, 512
    say("mul_mat_id-invalid", qtype, T)
    raw = synth.weights(qtype, E * M, K, seed=151)
    ids = synth.moe_ids(T, E, n_used, seed=152)
    ids[0, 1] = -1
    if T > 1:
        ids[1, 0] = E                                             # out of range
        ids[T - 1, :] = [-7, E + 3, -1, E]                        # a whole token of invalid ids
    x = synth.activations(T, K, seed=153).reshape(T, 1, K)
    w = sc.weights(qtype, raw, (K, M, E))
    y = sc.f32(np.full((T, n_used, M), 7.0, np.float32))          # dst holds non-zeros
    be.mul_mat_id(w, sc.f32(x), sc.i32(ids), y)
    if T > 1:
        with pytest.raises(qmm.QmmError, match="past the expert count"):
            be.synchronize()
    be.synchronize()
    got = be.get_f32(y).reshape(T, n_used, M)
    ref = orc.mul_mat_id(qtype, raw, M, K, E, x, ids)
    bad = (ids < 0) | (ids >= E)
    assert (got[bad] == 0).all()
    assert rel_err(got[~bad], ref[~bad]) <= TOL


def test_graph_route_shared_by_gate_and_up(be, sc, orc):
    """gate and up MUL_MAT_IDs with the same ids in one graph reuse one route (the second
    launches no routing); the down projection (ne11 = n_used) routes again"""
    E, n_used, M, K, T = 32, 4, 64, 512, 9
    say("graph-route-cache")
    rg, ru = synth.weights(qmm.Q4_K, E * M, K, 161), synth.weights(qmm.Q4_K, E * M, K, 162)
    rd = synth.weights(qmm.Q4_K, E * K, M * 4, 163)               # down: [4M, K, E] (K' = 4 M)
    ids = synth.moe_ids(T, E, n_used, seed=164)
    ids[2, 1] = -1
    wg, wu = sc.weights(qmm.Q4_K, rg, (K, M, E)), sc.weights(qmm.Q4_K, ru, (K, M, E))
    wd = sc.weights(qmm.Q4_K, rd, (4 * M, K, E))
    x = synth.activations(T, K, seed=165).reshape(T, 1, K)
    xd = synth.activations(T * n_used, 4 * M, seed=166).reshape(T, n_used, 4 * M)
    xt, xdt, it = sc.f32(x), sc.f32(xd), sc.i32(ids)
    yg, yu = sc.f32(np.full((T, n_used, M), 3.0, np.float32)), sc.f32(np.full((T, n_used, M), 3.0, np.float32))
    yd = sc.f32(np.full((T, n_used, K), 3.0, np.float32))
    be.graph_compute([(qmm.OP_MUL_MAT_ID, wg, xt, it, yg), (qmm.OP_MUL_MAT_ID, wu, xt, it, yu),
                      (qmm.OP_MUL_MAT_ID, wd, xdt, it, yd)])
    be.synchronize()
    bad = ids < 0
    for y, raw, xx, m, k in ((yg, rg, x, M, K), (yu, ru, x, M, K), (yd, rd, xd, K, 4 * M)):
        got = be.get_f32(y).reshape(T, n_used, m)
        ref = orc.mul_mat_id(qmm.Q4_K, raw, m, k, E, xx, ids)
        assert (got[bad] == 0).all()
        assert rel_err(got[~bad], ref[~bad]) <= TOL


@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q4_0])
def test_graph_shared_src1_new_ids(be, sc, orc, qtype):
    """MUL_MAT_IDs in one graph on the same src1 with other ids: the activations are quantized
    once (route and quantization in one launch), the later nodes route alone"""
    E, n_used, M, K, T = 16, 3, 64, 512, 7
    say("graph-src1-new-ids", qtype)
    raws = [synth.weights(qtype, E * M, K, 191 + i) for i in range(3)]
    idss = [synth.moe_ids(T, E, n_used, seed=194 + i) for i in range(2)]
    idss[1][3, 0] = -1
    ws = [sc.weights(qtype, r, (K, M, E)) for r in raws]
    x = synth.activations(T, K, seed=196).reshape(T, 1, K)
    xt = sc.f32(x)
    its = [sc.i32(i) for i in idss]
    ys = [sc.f32(np.full((T, n_used, M), 3.0, np.float32)) for _ in range(3)]
    order = [(0, 0), (1, 1), (2, 0)]                             # weights, ids: back to the first ids
    be.graph_compute([(qmm.OP_MUL_MAT_ID, ws[w], xt, its[i], ys[n]) for n, (w, i) in enumerate(order)])
    be.synchronize()
    for n, (w, i) in enumerate(order):
        got = be.get_f32(ys[n]).reshape(T, n_used, M)
        ref = orc.mul_mat_id(qtype, raws[w], M, K, E, x, idss[i])
        bad = idss[i] < 0
        assert (got[bad] == 0).all()
        assert rel_err(got[~bad], ref[~bad]) <= TOL, n


@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q4_0, qmm.Q6_K])
@pytest.mark.parametrize("T,E", [(1, 16), (4, 16), (40, 16), (300, 64), (40, 512)])
def test_mul_mat_id_glu(be, sc, orc, qtype, T, E):
    """MUL_MAT_ID gate, MUL_MAT_ID up and the GLU in one call (one route, one GEMV launch over
    both stacks: the two-pass form into a scratch plus the GLU kernel at few tasks, the
    in-work-group GLU at many - T = 300 on 64 experts and T = 40 on 512 pass the 1024
    work-group mark); invalid ids give zero rows"""
    from oracle import glu as G
    n_used, M, K = 4, 130, 512
    say("mul_mat_id_glu", qtype, T)
    rg, ru = synth.weights(qtype, E * M, K, seed=171), synth.weights(qtype, E * M, K, seed=172)
    ids = synth.moe_ids(T, E, n_used, seed=173)
    ids[0, 2] = -1
    if T > 1:
        ids[1, 0] = E + 2
    x = synth.activations(T, K, seed=174).reshape(T, 1, K)
    wg, wu = sc.weights(qtype, rg, (K, M, E)), sc.weights(qtype, ru, (K, M, E))
    y = sc.f32(np.full((T, n_used, M), 5.0, np.float32))
    be.mul_mat_id_glu(wg, wu, sc.f32(x), sc.i32(ids), y, qmm.GLU_SWIGLU)
    if T > 1:                                                     # the id E + 2 is reported
        with pytest.raises(qmm.QmmError, match="past the expert count"):
            be.synchronize()
    be.synchronize()
    assert be.last_path().startswith("glu-gemv-id")
    got = be.get_f32(y).reshape(T, n_used, M)
    ref = G.glu(qmm.GLU_SWIGLU, orc.mul_mat_id(qtype, rg, M, K, E, x, ids), orc.mul_mat_id(qtype, ru, M, K, E, x, ids))
    bad = (ids < 0) | (ids >= E)
    assert (got[bad] == 0).all()
    assert rel_err(got[~bad], ref[~bad]) <= TOL


def test_mul_mat_id_glu_per_slot_src1(be, sc, orc):
    """src1 [K, n_used, T] (one row per slot) and GEGLU"""
    from oracle import glu as G
    E, n_used, M, K, T = 8, 3, 64, 256, 5
    say("mul_mat_id_glu ne11=n_used")
    rg, ru = synth.weights(qmm.Q4_K, E * M, K, seed=181), synth.weights(qmm.Q4_K, E * M, K, seed=182)
    ids = synth.moe_ids(T, E, n_used, seed=183)
    x = synth.activations(T * n_used, K, seed=184).reshape(T, n_used, K)
    wg, wu = sc.weights(qmm.Q4_K, rg, (K, M, E)), sc.weights(qmm.Q4_K, ru, (K, M, E))
    y = sc.empty_f32((M, n_used, T))
    be.mul_mat_id_glu(wg, wu, sc.f32(x), sc.i32(ids), y, qmm.GLU_GEGLU)
    be.synchronize()
    got = be.get_f32(y).reshape(T, n_used, M)
    ref = G.glu(qmm.GLU_GEGLU, orc.mul_mat_id(qmm.Q4_K, rg, M, K, E, x, ids), orc.mul_mat_id(qmm.Q4_K, ru, M, K, E, x, ids))
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("op,bcast,qtype", [(qmm.GLU_SWIGLU, True, qmm.Q4_K), (qmm.GLU_GEGLU, False, qmm.Q4_K),
                                            (qmm.GLU_REGLU, True, qmm.Q4_K), (qmm.GLU_SWIGLU, False, qmm.Q5_K),
                                            (qmm.GLU_GEGLU, True, qmm.IQ4_XS), (qmm.GLU_SWIGLU, True, qmm.Q6_K)])
def test_mul_mat_id_glu_grouped_gemm(be, sc, orc, monkeypatch, op, bcast, qtype):
    """MUL_MAT_ID gate + up + GLU on the grouped GEMM (experts averaging >= 32 pairs): one route
    and quantization, the gate product into a scratch at dst's offsets, the up product storing
    act(gate) * up; ragged (100 rows, 3 of 8 experts without pairs, pair counts not a multiple of
    64), negative ids give zero rows, an id past the expert count is reported; the same op on the
    GEMV tasks agrees"""
    from oracle import glu as G
    E, n_used, M, K, T = 8, 3, 100, 1280, 300
    say("mul_mat_id_glu grouped gemm", op, bcast, qtype)
    rg, ru = synth.weights(qtype, E * M, K, seed=191), synth.weights(qtype, E * M, K, seed=192)
    g = np.random.default_rng(193)
    ids = np.stack([g.choice([0, 2, 4, 5, 6], size=n_used, replace=False) for _ in range(T)]).astype(np.int32)
    ids[7, 1] = -1
    ids[11, 0] = -1
    ne11 = 1 if bcast else n_used
    x = synth.activations(T * ne11, K, seed=194).reshape(T, ne11, K)
    wg, wu = sc.weights(qtype, rg, (K, M, E)), sc.weights(qtype, ru, (K, M, E))
    y = sc.f32(np.full((T, n_used, M), 5.0, np.float32))
    be.mul_mat_id_glu(wg, wu, sc.f32(x), sc.i32(ids), y, op)
    be.synchronize()
    assert be.last_path() == "glu-gemm-id-stream"
    got = be.get_f32(y).reshape(T, n_used, M)
    ref = G.glu(op, orc.mul_mat_id(qtype, rg, M, K, E, x, ids), orc.mul_mat_id(qtype, ru, M, K, E, x, ids))
    assert not got[7, 1].any() and not got[11, 0].any()
    bad = ids < 0
    assert rel_err(got[~bad], ref[~bad]) <= TOL
    monkeypatch.setenv("QMM_MOE_GEMM_MIN", "0")
    y2 = sc.empty_f32((M, n_used, T))
    be.mul_mat_id_glu(wg, wu, sc.f32(x), sc.i32(ids), y2, op)
    be.synchronize()
    assert be.last_path().startswith("glu-gemv-id")
    assert rel_err(got, be.get_f32(y2).reshape(T, n_used, M)) <= TOL
    monkeypatch.delenv("QMM_MOE_GEMM_MIN")
    over = ids.copy()
    over[5, 2] = E + 1
    be.mul_mat_id_glu(wg, wu, sc.f32(x), sc.i32(over), sc.empty_f32((M, n_used, T)), op)
    assert be.last_path() == "glu-gemm-id-stream"
    with pytest.raises(qmm.QmmError, match="past the expert count"):
        be.synchronize()


def test_downgrade_keys(sc, orc, monkeypatch):
    """the downgrade export counts per key: Q5_K at 4 columns runs on the v_dot4 GEMV (no MFMA
    form), Q4_K at 40 columns takes two weight passes on the MFMA GEMV; a product on its
    promised path adds nothing (the fused kernel, which takes these small products at 1-16
    columns, switched off)"""
    monkeypatch.setenv("QMM_GEMV_FQ_SMALL_TG", "0")
    monkeypatch.setenv("QMM_GEMV_FQS", "0")
    say("downgrades")
    with qmm.Backend(0) as b2:
        bufs = []

        def run(qtype, M, K, N):
            w = b2.new_tensor(qtype, (K, M))
            b2.set_tensor(w, synth.weights(qtype, M, K, 1))
            x = b2.new_tensor(qmm.F32, (K, N))
            b2.set_tensor(x, synth.activations(N, K, 2).view(np.uint8).ravel())
            y = b2.new_tensor(qmm.F32, (M, N))
            b2.mul_mat(w, x, y)
            bufs.extend([w, x, y])

        run(qmm.Q4_K, 128, 512, 1)
        assert b2.downgrades() == (0, {})
        run(qmm.Q5_K, 128, 512, 4)
        run(qmm.Q5_K, 128, 512, 5)
        run(qmm.Q4_K, 128, 512, 40)
        b2.synchronize()
        n, keys = b2.downgrades()
        assert keys == {"src=qmm op=MUL_MAT type=Q5_K k=512 cols=2-8 path=gemv reason=no-mfma-gemv": 2,
                        "src=qmm op=MUL_MAT type=Q4_K k=512 cols=33-128 path=gemv-mfma reason=several-weight-passes": 1}
        assert n == 3
        # the shared-tile GEMM when the streaming one is switched off (QMM_GEMM3_SBS=0 for Q5_K);
        # Q6_K streams (no key)
        monkeypatch.setenv("QMM_GEMM3_SBS", "0")
        run(qmm.Q5_K, 128, 512, 512)
        monkeypatch.delenv("QMM_GEMM3_SBS")
        run(qmm.Q6_K, 128, 512, 512)
        b2.synchronize()
        n, keys = b2.downgrades()
        assert keys["src=qmm op=MUL_MAT type=Q5_K k=512 cols=129+ path=gemm-mfma reason=no-streaming-gemm"] == 1
        assert not any("type=Q6_K" in k and "no-streaming-gemm" in k for k in keys), keys
        # MUL_MAT_ID on route tasks: 16 experts, 80 tokens x 8 used = 40 pairs an expert (each expert's
        # weights stream once per 8-pair task), past the grouped GEMM's 32-pair threshold: Q6_K's
        # grouped GEMM needs K >= 512 (K = 256 here), Q8_0 has none (K = 512)
        E, T, k, M = 16, 80, 8, 64
        for qt, name, why, K in ((qmm.Q6_K, "Q6_K", "grouped-gemm-needs-k-512", 256),
                                 (qmm.Q8_0, "Q8_0", "no-grouped-gemm-for-type", 512)):
            w = b2.new_tensor(qt, (K, M, E))
            b2.set_tensor(w, synth.weights(qt, M * E, K, 3))
            x = b2.new_tensor(qmm.F32, (K, 1, T))
            b2.set_tensor(x, synth.activations(T, K, 4).view(np.uint8).ravel())
            ids = b2.new_tensor(qmm.I32, (k, T))
            b2.set_tensor(ids, synth.moe_ids(T, E, k, 5).view(np.uint8).ravel())
            y = b2.new_tensor(qmm.F32, (M, k, T))
            b2.mul_mat_id(w, x, ids, y)
            bufs.extend([w, x, ids, y])
            b2.synchronize()
            n, keys = b2.downgrades()
            path = b2.last_path()
            assert keys[f"src=qmm op=MUL_MAT_ID type={name} k={K} pairs/expert=33-128 path={path} "
                        "reason=expert-weights-per-8-pair-task"] == 1
            assert keys[f"src=qmm op=MUL_MAT_ID type={name} k={K} pairs/expert=33-128 path={path} "
                        f"reason={why}"] == 1



# ------------------------------------------------------------------ the fused-quantization GEMV
@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("N", [1, 2])
@pytest.mark.parametrize("M,K", [(300, 2048), (1, 256), (65, 5120), (63, 768), (130, 4352)])
def test_fused_gemv(be, sc, orc, monkeypatch, qtype, N, M, K):
    """k_gemv_fq (each wave quantizes its own groups; K split only inside the work-group) on
    every type, forced onto small shapes; K = 4352 takes 17 groups, more than the work-group's 16
    waves"""
    monkeypatch.setenv("QMM_GEMV_FQ_MIN_WAVES", "1")
    say("fused", qtype, M, K, N)
    got, ref = run_mul_mat(be, sc, orc, qtype, M, K, N, seed=201)
    assert be.last_path() == "gemv-fq"
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("qtype", [qmm.Q4_0, qmm.Q8_0, qmm.IQ4_NL])
@pytest.mark.parametrize("K", [640, 416])
def test_fused_gemv_partial_group(be, sc, orc, monkeypatch, qtype, K):
    monkeypatch.setenv("QMM_GEMV_FQ_MIN_WAVES", "1")
    say("fused partial group", qtype, K)
    got, ref = run_mul_mat(be, sc, orc, qtype, 200, K, 2, seed=202)
    assert be.last_path() == "gemv-fq"
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q4_0, qmm.Q6_K])
def test_fused_gemv_broadcast_strides_and_split_path(be, sc, orc, monkeypatch, qtype):
    """broadcast batches, a strided src1 view and a padded dst on the fused kernel; the same
    product on the pre-pass path (QMM_GEMV_FUSED=0) agrees"""
    monkeypatch.setenv("QMM_GEMV_FQ_MIN_WAVES", "1")
    say("fused broadcast", qtype)
    K, M, N = 512, 80, 2
    raw = synth.weights(qtype, 2 * M, K, seed=203)
    w = sc.weights(qtype, raw, (K, M, 2))
    x = synth.activations(8 * N, K, seed=204).reshape(4, 2 * N, K)        # every other column used
    xt = sc.f32(x)
    xv = qmm.Tensor(xt.buf, qmm.F32, (K, N, 4), nb=(4, 8 * K, 8 * K * N, 8 * K * N * 4))
    ypad = sc.empty_f32((M + 5, N, 4))
    yv = qmm.Tensor(ypad.buf, qmm.F32, (M, N, 4), nb=(4, 4 * (M + 5), 4 * (M + 5) * N, 4 * (M + 5) * N * 4))
    be.mul_mat(w, xv, yv)
    be.synchronize()
    assert be.last_path() == "gemv-fq"
    got = be.get_f32(ypad).reshape(4, N, M + 5)[:, :, :M].copy()
    rb = synth.row_bytes(qtype, K) * M
    for i2 in range(4):
        assert rel_err(got[i2], orc.mul_mat(qtype, raw[(i2 // 2) * rb:(i2 // 2 + 1) * rb], M, K, x[i2, 0::2])) <= TOL
    monkeypatch.setenv("QMM_GEMV_FUSED", "0")
    be.mul_mat(w, xv, yv)
    be.synchronize()
    assert be.last_path() == "gemv"
    assert rel_err(be.get_f32(ypad).reshape(4, N, M + 5)[:, :, :M], got) <= TOL


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("M,K,N,W", [(300, 2048, 1, 4), (130, 5120, 2, 3), (65, 4352, 1, 1), (64, 768, 2, 2),
                                     (1, 768, 1, 1)])
def test_fused_gemv_split(be, sc, orc, monkeypatch, qtype, M, K, N, W):
    """K split over work-groups of the fused kernel, their sums met in the exchange tree: KS = 2;
    20 groups over 7 slices of 3 waves (an odd KS, an idle last wave); 17 one-group slices; 3
    groups over 2 slices of 2 waves; a one-row matrix.  Twice on the same weights with new
    activations: the tree's slots are empty again after every launch"""
    monkeypatch.setenv("QMM_GEMV_FQS", "1")
    monkeypatch.setenv("QMM_GEMV_FQS_W", str(W))
    monkeypatch.setenv("QMM_GEMV_FQ_SMALL_TG", "0")
    say("fused split", qtype, M, K, N, W)
    raw = synth.weights(qtype, M, K, seed=211)
    w = sc.weights(qtype, raw, (K, M))
    xt, y = sc.f32(np.zeros((N, K), np.float32)), sc.empty_f32((M, N))
    G = -(-K // 256)
    for seed in (212, 213):
        x = synth.activations(N, K, seed=seed)
        be.set_tensor(xt, x.view(np.uint8).ravel())
        be.mul_mat(w, xt, y)
        be.synchronize()
        assert be.last_path() == "gemv-fq"
        assert qmm.describe_mul_mat(w, xt, y)["k_slices"] == -(-G // W)
        assert rel_err(be.get_f32(y).reshape(N, M), orc.mul_mat(qtype, raw, M, K, x)) <= TOL, seed


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("N", [3, 5, 8, 12])
def test_fused_gemv_small_many_columns(be, sc, orc, qtype, N):
    """small products (8 groups along K, 5 tiles) of 3-16 columns take the fused kernel as
    2-column tasks (one launch instead of the pre-pass and the MFMA GEMV; Q5_K's GEMM, which
    MUL_MAT picks first, starts at 16 columns)"""
    say("fused small many columns", qtype, N)
    got, ref = run_mul_mat(be, sc, orc, qtype, 300, 2048, N, seed=221)
    assert be.last_path() == "gemv-fq"
    assert rel_err(got, ref) <= TOL


def test_fused_gemv_small_many_columns_batches(be, sc, orc):
    """5 columns (2-column tasks, the last with one) over broadcast batches: two matrices, four
    batches"""
    say("fused small many columns batches")
    qtype, K, M, N = qmm.Q4_K, 512, 80, 5
    raw = synth.weights(qtype, 2 * M, K, seed=222)
    w = sc.weights(qtype, raw, (K, M, 2))
    x = synth.activations(4 * N, K, seed=223).reshape(4, N, K)
    xt = sc.f32(x)
    y = sc.empty_f32((M, N, 4))
    be.mul_mat(w, xt, y)
    be.synchronize()
    assert be.last_path() == "gemv-fq"
    got = be.get_f32(y).reshape(4, N, M)
    rb = synth.row_bytes(qtype, K) * M
    for i2 in range(4):
        assert rel_err(got[i2], orc.mul_mat(qtype, raw[(i2 // 2) * rb:(i2 // 2 + 1) * rb], M, K, x[i2])) <= TOL


@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q4_0, qmm.Q6_K])
def test_fused_gemv_split_broadcast(be, sc, orc, monkeypatch, qtype):
    """the K-split fused kernel over broadcast batches with a strided src1 view and a padded dst
    (each batch's tiles meet in their own tree slots)"""
    monkeypatch.setenv("QMM_GEMV_FQS", "1")
    monkeypatch.setenv("QMM_GEMV_FQS_W", "1")
    monkeypatch.setenv("QMM_GEMV_FQ_SMALL_TG", "0")
    say("fused split broadcast", qtype)
    K, M, N = 512, 80, 2
    raw = synth.weights(qtype, 2 * M, K, seed=214)
    w = sc.weights(qtype, raw, (K, M, 2))
    x = synth.activations(8 * N, K, seed=215).reshape(4, 2 * N, K)
    xt = sc.f32(x)
    xv = qmm.Tensor(xt.buf, qmm.F32, (K, N, 4), nb=(4, 8 * K, 8 * K * N, 8 * K * N * 4))
    ypad = sc.empty_f32((M + 5, N, 4))
    yv = qmm.Tensor(ypad.buf, qmm.F32, (M, N, 4), nb=(4, 4 * (M + 5), 4 * (M + 5) * N, 4 * (M + 5) * N * 4))
    be.mul_mat(w, xv, yv)
    be.synchronize()
    assert be.last_path() == "gemv-fq"
    got = be.get_f32(ypad).reshape(4, N, M + 5)[:, :, :M]
    rb = synth.row_bytes(qtype, K) * M
    for i2 in range(4):
        assert rel_err(got[i2], orc.mul_mat(qtype, raw[(i2 // 2) * rb:(i2 // 2 + 1) * rb], M, K, x[i2, 0::2])) <= TOL


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("T", [1, 4, 15])
@pytest.mark.parametrize("bcast", [True, False])
def test_mul_mat_id_direct(be, sc, orc, qtype, T, bcast):
    """MUL_MAT_ID below 16 tokens: each (slot, token) pair reads its expert id in the fused GEMV
    (no route launch); a negative id writes a zero row, an id past the stack too and is reported
    by synchronize"""
    E, n_used, M, K = 16, 4, 96, 512
    say("mul_mat_id direct", qtype, T, bcast)
    raw = synth.weights(qtype, E * M, K, seed=205)
    ids = synth.moe_ids(T, E, n_used, seed=206)
    ids[0, 1] = -1
    if T > 1:
        ids[T - 1, 3] = E + 1
    ne11 = 1 if bcast else n_used
    x = synth.activations(T * ne11, K, seed=207).reshape(T, ne11, K)
    w = sc.weights(qtype, raw, (K, M, E))
    y = sc.f32(np.full((T, n_used, M), 9.0, np.float32))
    be.mul_mat_id(w, sc.f32(x), sc.i32(ids), y)
    assert be.last_path() == "gemv-id-fq"
    if T > 1:
        with pytest.raises(qmm.QmmError, match="past the expert count"):
            be.synchronize()
    be.synchronize()
    got = be.get_f32(y).reshape(T, n_used, M)
    bad = (ids < 0) | (ids >= E)
    assert (got[bad] == 0).all()
    assert rel_err(got[~bad], orc.mul_mat_id(qtype, raw, M, K, E, x, ids)[~bad]) <= TOL


@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q4_0, qmm.Q6_K])
@pytest.mark.parametrize("T", [1, 4, 19])
def test_mul_mat_id_route_and_direct_agree(be, sc, orc, monkeypatch, qtype, T):
    """the same MUL_MAT_ID on the route (QMM_MOE_DIRECT_T=0) and on the pairs
    (QMM_MOE_DIRECT_T=1000), gate/up + GLU included"""
    from oracle import glu as G
    E, n_used, M, K = 32, 6, 130, 512
    say("mul_mat_id route vs direct", qtype, T)
    rg, ru = synth.weights(qtype, E * M, K, seed=208), synth.weights(qtype, E * M, K, seed=209)
    ids = synth.moe_ids(T, E, n_used, seed=210)
    x = synth.activations(T, K, seed=211).reshape(T, 1, K)
    wg, wu = sc.weights(qtype, rg, (K, M, E)), sc.weights(qtype, ru, (K, M, E))
    xt, it = sc.f32(x), sc.i32(ids)
    outs = {}
    for direct in ("0", "1000"):
        monkeypatch.setenv("QMM_MOE_DIRECT_T", direct)
        y, yg = sc.empty_f32((M, n_used, T)), sc.empty_f32((M, n_used, T))
        be.mul_mat_id(wg, xt, it, y)
        p1 = be.last_path()
        be.mul_mat_id_glu(wg, wu, xt, it, yg, qmm.GLU_SWIGLU)
        p2 = be.last_path()
        be.synchronize()
        assert (p1 == "gemv-id-fq") == (direct != "0") and (p2 == "glu-gemv-id-fq") == (direct != "0"), (p1, p2)
        outs[direct] = (be.get_f32(y).reshape(T, n_used, M), be.get_f32(yg).reshape(T, n_used, M))
    ref = orc.mul_mat_id(qtype, rg, M, K, E, x, ids)
    refg = G.glu(qmm.GLU_SWIGLU, ref, orc.mul_mat_id(qtype, ru, M, K, E, x, ids))
    for direct, (a, b) in outs.items():
        assert rel_err(a, ref) <= TOL, direct
        assert rel_err(b, refg) <= TOL, direct


@pytest.mark.parametrize("op", GLU_OPS)
@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q5_K, qmm.IQ4_NL])
def test_mul_mat_glu_fused_kernel(be, sc, orc, monkeypatch, op, qtype):
    """gate/up + GLU on the fused kernel: each work-group streams the gate tile, then the up tile,
    and stores act(gate) * up"""
    monkeypatch.setenv("QMM_GEMV_FQ_MIN_WAVES", "1")
    say("glu fused kernel", op, qtype)
    got, ref = glu_case(be, sc, orc, qtype, qtype, 200, 1024, 2, op, seed=212, batches=(2, 1))
    assert be.last_path() == "glu-fused-gemv-fq"
    assert rel_err(got, ref) <= TOL
