"""Pins of the CPU oracle (oracle/qmm_oracle.c) against what does not come from
the oracle itself: hand-derived known answers from ggml's block formats,
numpy's IEEE binary16 conversions, the reference's kvalues_iq4nl literal,
exact-representability invariants and the textbook identity
dot(w, q8(x)) == sum(dequant(w) * dequant(q8(x))) evaluated in fp64.
CPU only."""
import numpy as np
import pytest

import oracle as O


def f16(v) -> bytes:
    return np.float16(v).tobytes()


# ---------------------------------------------------------------- fp16
def test_fp16_to_fp32_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.fp16_to_fp32(int(b)) for b in bits], np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def test_fp32_to_fp16_round_to_nearest_even(orc):
    g = np.random.default_rng(1)
    xs = np.concatenate([
        g.standard_normal(20000).astype(np.float32) * np.float32(0.02),
        (g.random(5000) * 7e-5).astype(np.float32),            # half subnormals and the normal boundary
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 6e-8, 2.9e-8, 3e-8], np.float32),
    ])
    # exact ties: halfway between two fp16 values
    h = np.arange(0x3C00, 0x3C40, dtype=np.uint16).view(np.float16).astype(np.float32)
    xs = np.concatenate([xs, (h[:-1] + h[1:]) / 2])
    ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([orc.fp32_to_fp16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- dequant KATs
def test_q4_0_nibble_positions_and_offset(orc):
    # d = 1.0: weight j (j < 16) is the low nibble of byte j minus 8,
    # weight j + 16 the high nibble minus 8
    for v in range(256):
        blk = f16(1.0) + bytes([v] * 16)
        y = orc.dequantize(O.Q4_0, np.frombuffer(blk, np.uint8), 32)
        assert np.all(y[:16] == (v & 15) - 8) and np.all(y[16:] == (v >> 4) - 8)
    qs = bytes(range(0, 256, 16))      # low nibble 0 everywhere, high nibble = j
    y = orc.dequantize(O.Q4_0, np.frombuffer(f16(0.5) + qs, np.uint8), 32)
    assert list(y[:16]) == [-4.0] * 16 and list(y[16:]) == [0.5 * (j - 8) for j in range(16)]


def test_q8_0_values(orc):
    qs = np.arange(-128, 128, dtype=np.int8)
    raw = b"".join(f16(0.25) + qs[32 * i:32 * i + 32].tobytes() for i in range(8))
    y = orc.dequantize(O.Q8_0, np.frombuffer(raw, np.uint8), 256)
    assert np.array_equal(y, qs.astype(np.float32) * 0.25)


def _q4k_block(d, dmin, scales12, qs128):
    return np.frombuffer(f16(d) + f16(dmin) + np.asarray(scales12, np.uint8).tobytes()
                         + np.asarray(qs128, np.uint8).tobytes(), np.uint8)


def test_q4_K_scale_min_unpack_known_answer(orc):
    # hand-derived from get_scale_min_k4 (P01:2164-2176):
    # j < 4: sc = q[j] & 63, m = q[j+4] & 63
    # j >= 4: sc = (q[j+4] & 15) | (q[j-4] >> 6) << 4, m = (q[j+4] >> 4) | (q[j] >> 6) << 4
    sc12 = [0xC1, 0x02, 0x03, 0x04, 0x45, 0x06, 0x07, 0x08, 0x9A, 0xBC, 0xDE, 0xF0]
    sc_exp = [1, 2, 3, 4, 58, 12, 14, 0]
    m_exp = [5, 6, 7, 8, 25, 11, 13, 15]
    # all codes 0: y = -dmin * m ; all codes 1: y = d * sc - dmin * m
    y0 = orc.dequantize(O.Q4_K, _q4k_block(1.0, 1.0, sc12, [0x00] * 128), 256)
    y1 = orc.dequantize(O.Q4_K, _q4k_block(1.0, 1.0, sc12, [0x11] * 128), 256)
    for j in range(8):
        assert np.all(y0[32 * j:32 * j + 32] == -m_exp[j]), j
        assert np.all(y1[32 * j:32 * j + 32] == sc_exp[j] - m_exp[j]), j


def test_q4_K_code_positions(orc):
    # byte l of chunk c: low nibble -> weight 64c + l, high nibble -> 64c + 32 + l
    sc12 = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]   # every sub-block scale 1, min 0
    for c in range(4):
        for l in (0, 7, 31):
            qs = [0] * 128
            qs[32 * c + l] = 0x5A
            y = orc.dequantize(O.Q4_K, _q4k_block(2.0, 3.0, sc12, qs), 256)
            nz = np.nonzero(y)[0]
            assert list(nz) == sorted([64 * c + l, 64 * c + 32 + l])
            assert y[64 * c + l] == 2.0 * 10 and y[64 * c + 32 + l] == 2.0 * 5


def test_q4_K_rounding_only_in_the_subtract(orc):
    # d1 * q is exact; the single rounding is d1*q - m1 in fp32 (no fused multiply-add)
    g = np.random.default_rng(3)
    for _ in range(200):
        d = np.float16(abs(g.normal(0, 0.02)))
        dmin = np.float16(abs(g.normal(0, 0.02)))
        sc12 = g.integers(0, 256, 12)
        qs = g.integers(0, 256, 128)
        y = orc.dequantize(O.Q4_K, _q4k_block(d, dmin, sc12, qs), 256)
        # unit scales expose the integer sub-scale and min exactly (sc - m and -m)
        y1 = orc.dequantize(O.Q4_K, _q4k_block(1.0, 1.0, sc12, [0x11] * 128), 256)
        y0 = orc.dequantize(O.Q4_K, _q4k_block(1.0, 1.0, sc12, [0x00] * 128), 256)
        for w in range(256):
            c, r = divmod(w, 64)
            code = (qs[32 * c + r % 32] >> (4 * (r >= 32))) & 15
            m = -y0[w]
            sc = y1[w] + m
            d1 = np.float32(d) * np.float32(sc)           # exact (17 significant bits)
            m1 = np.float32(dmin) * np.float32(m)         # exact
            exp = np.float32(d1 * np.float32(code)) - m1  # d1 * code exact; one rounding
            assert y[w] == exp


def _q6k_block(ql, qh, scales, d):
    return np.frombuffer(np.asarray(ql, np.uint8).tobytes() + np.asarray(qh, np.uint8).tobytes()
                         + np.array(scales, np.int8).tobytes() + f16(d), np.uint8)


def test_q6_K_single_code_positions(orc):
    # weight w = 128n + 32g + l: ql[64n + l + 32 (g & 1)] (low nibble g < 2, high g >= 2),
    # qh[32n + l] bits 2g..2g+1, scale index 8n + 2g + l // 16 (dequantize_row_q6_K)
    scales = list(range(1, 17))
    for w in (0, 15, 16, 31, 32, 47, 64, 95, 96, 127, 128, 160, 200, 255):
        n, r = divmod(w, 128)
        g, l = divmod(r, 32)
        ql = [0] * 128
        qh = [0] * 64
        ql[64 * n + l + 32 * (g & 1)] = 0x0F if g < 2 else 0xF0
        qh[32 * n + l] = 3 << (2 * g)
        y = orc.dequantize(O.Q6_K, _q6k_block(ql, qh, scales, 1.0), 256)
        for v in range(256):
            nv, rv = divmod(v, 128)
            gv, lv = divmod(rv, 32)
            sc = scales[8 * nv + 2 * gv + lv // 16]
            assert y[v] == sc * (31 if v == w else -32), (w, v)


def test_iq4_xs_codebook_matches_reference_literal(orc):
    # P01:3335-3337: kvalues_iq4nl
    assert orc.kvalues() == [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def test_iq4_xs_scales_and_positions(orc):
    # ls(ib) = ((scales_l[ib/2] >> 4 (ib%2)) & 15) | ((scales_h >> 2 ib) & 3) << 4
    scales_h = 0b11_10_01_00_11_10_01_00      # ib: 0->0, 1->1, 2->2, 3->3, 4->0, 5->1, 6->2, 7->3
    scales_l = [0x21, 0x43, 0x65, 0x87]       # low nibble ib even, high ib odd: 1, 2, 3, ..., 8
    ls = [(k + 1) | (h << 4) for k, h in zip(range(8), [0, 1, 2, 3, 0, 1, 2, 3])]
    kv = orc.kvalues()
    for ib in range(8):
        for j in (0, 5, 15):
            qs = [0x88] * 128          # code 8 -> kv = 1 everywhere
            qs[16 * ib + j] = 0x3C     # low nibble 12 -> weight 32ib + j, high 3 -> 32ib + 16 + j
            raw = f16(1.0) + np.uint16(scales_h).tobytes() + bytes(scales_l) + bytes(qs)
            y = orc.dequantize(O.IQ4_XS, np.frombuffer(raw, np.uint8), 256)
            exp = np.array([ls[v // 32] - 32 for v in range(256)], np.float32)
            exp[16 * 0 + 32 * ib + j] *= kv[12]
            exp[32 * ib + 16 + j] *= kv[3]
            assert np.array_equal(y, exp), (ib, j)


def test_iq4_nl_known_answer_and_equals_iq4_xs_at_unit_scales(orc):
    # weight j (j < 16) = d * kv[low nibble of byte j], j + 16: d * kv[high nibble]
    kv = orc.kvalues()
    for v in (0x00, 0x98, 0xF0, 0x3C, 0xFF):
        y = orc.dequantize(O.IQ4_NL, np.frombuffer(f16(0.5) + bytes([v] * 16), np.uint8), 32)
        assert np.all(y[:16] == 0.5 * kv[v & 15]) and np.all(y[16:] == 0.5 * kv[v >> 4])
    # an IQ4_XS super-block with every ls = 33 (scale ls - 32 = 1) is 8 IQ4_NL blocks of its d
    g = np.random.default_rng(8)
    for _ in range(20):
        d = np.float16(abs(g.normal(0, 0.02)))
        qs = g.integers(0, 256, 128, dtype=np.uint8)
        xs = f16(d) + np.uint16(0b10_10_10_10_10_10_10_10).tobytes() + bytes([0x11] * 4) + qs.tobytes()
        nl = b"".join(f16(d) + qs[16 * i:16 * i + 16].tobytes() for i in range(8))
        assert np.array_equal(orc.dequantize(O.IQ4_XS, np.frombuffer(xs, np.uint8), 256),
                              orc.dequantize(O.IQ4_NL, np.frombuffer(nl, np.uint8), 256))


def _q5k_block(d, dmin, scales12, qh32, qs128):
    return np.frombuffer(f16(d) + f16(dmin) + np.asarray(scales12, np.uint8).tobytes()
                         + np.asarray(qh32, np.uint8).tobytes() + np.asarray(qs128, np.uint8).tobytes(), np.uint8)


def test_q5_K_without_fifth_bits_is_q4_K(orc):
    g = np.random.default_rng(9)
    for _ in range(50):
        d, dmin = np.float16(abs(g.normal(0, 0.02))), np.float16(abs(g.normal(0, 0.02)))
        sc12, qs = g.integers(0, 256, 12), g.integers(0, 256, 128)
        assert np.array_equal(orc.dequantize(O.Q5_K, _q5k_block(d, dmin, sc12, [0] * 32, qs), 256),
                              orc.dequantize(O.Q4_K, _q4k_block(d, dmin, sc12, qs), 256))


def test_q5_K_fifth_bit_positions(orc):
    # qh[l] bit 2c adds 16 to weight 64c + l (low nibble), bit 2c + 1 to weight 64c + 32 + l
    sc12 = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]   # every sub-block scale 1, min 0
    for c in range(4):
        for hi in (0, 1):
            for l in (0, 13, 31):
                qh = [0] * 32
                qh[l] = 1 << (2 * c + hi)
                y = orc.dequantize(O.Q5_K, _q5k_block(2.0, 3.0, sc12, qh, [0] * 128), 256)
                assert list(np.nonzero(y)[0]) == [64 * c + 32 * hi + l]
                assert y[64 * c + 32 * hi + l] == 2.0 * 16


def test_q5_K_rounding_only_in_the_subtract(orc):
    g = np.random.default_rng(10)
    for _ in range(100):
        d, dmin = np.float16(abs(g.normal(0, 0.02))), np.float16(abs(g.normal(0, 0.02)))
        sc12, qh, qs = g.integers(0, 256, 12), g.integers(0, 256, 32), g.integers(0, 256, 128)
        y = orc.dequantize(O.Q5_K, _q5k_block(d, dmin, sc12, qh, qs), 256)
        y1 = orc.dequantize(O.Q4_K, _q4k_block(1.0, 1.0, sc12, [0x11] * 128), 256)
        y0 = orc.dequantize(O.Q4_K, _q4k_block(1.0, 1.0, sc12, [0x00] * 128), 256)
        for w in range(256):
            c, r = divmod(w, 64)
            hi, l = divmod(r, 32)
            code = ((qs[32 * c + l] >> (4 * hi)) & 15) | (((qh[l] >> (2 * c + hi)) & 1) << 4)
            m = -y0[w]
            sc = y1[w] + m
            d1 = np.float32(d) * np.float32(sc)           # exact
            m1 = np.float32(dmin) * np.float32(m)         # exact
            assert y[w] == np.float32(d1 * np.float32(code)) - m1   # d1 * code exact (22 bits)


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.IQ4_NL])
def test_q4_0_q8_0_values_are_exact_multiples_of_d(orc, qtype):
    from arcint_amd import synth
    raw = synth.weights(qtype, 64, 256, seed=5)
    y = orc.dequantize(qtype, raw, 64 * 256).reshape(-1, 32)
    bs = 34 if qtype == O.Q8_0 else 18
    d = raw.reshape(-1, bs)[:, :2].copy().view(np.float16).astype(np.float64)
    q = y.astype(np.float64) / d
    assert np.array_equal(q, np.round(q))


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K, O.IQ4_NL, O.IQ4_XS])
def test_dequant_special_scales(orc, qtype):
    from arcint_amd import synth
    blck, bs = O.TYPES[qtype][:2]
    raw = synth.weights(qtype, 1, blck, seed=1).copy()
    doff = 208 if qtype == O.Q6_K else 0
    raw[doff:doff + 2] = np.frombuffer(f16(0.0), np.uint8)
    if qtype in (O.Q4_K, O.Q5_K):
        raw[2:4] = np.frombuffer(f16(0.0), np.uint8)
    assert np.all(orc.dequantize(qtype, raw, blck) == 0)
    raw[doff:doff + 2] = np.frombuffer(np.uint16(1).tobytes(), np.uint8)     # smallest subnormal d
    y = orc.dequantize(qtype, raw, blck)
    assert np.all(np.isfinite(y)) and np.any(y != 0)


# ---------------------------------------------------------------- quantizers
def test_q8_0_known_answers(orc):
    out = orc.quantize_q8_0(np.ones(32, np.float32))
    assert out[:2].view(np.float16)[0] == np.float16(1.0 / 127.0)
    assert np.all(out[2:].view(np.int8) == 127)
    # ties round half to even: amax 127 -> multiplier exactly 1
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5]
    q = orc.quantize_q8_0(x)[2:].view(np.int8)
    assert list(q[:9]) == [127, 0, 2, 2, 0, -2, -2, 4, 126]
    z = orc.quantize_q8_0(np.zeros(64, np.float32))
    assert not z.any()
    # d is amax / 127 rounded to fp16, the codes use 127 / amax unrounded
    x = np.linspace(-3.3, 2.2, 32).astype(np.float32)
    b = orc.quantize_q8_0(x)
    assert b[:2].view(np.float16)[0] == np.float16(np.float32(3.3) / np.float32(127))
    mul = np.float32(127) / np.float32(np.max(np.abs(x)))
    assert np.array_equal(b[2:].view(np.int8), np.rint(x * mul).astype(np.int8))


def _q8k_fields(b):
    d = b[0:4].view(np.float32)[0]
    qs = b[4:260].view(np.int8)
    bsums = b[260:292].view(np.int16)
    return d, qs, bsums


def test_q8_K_sign_of_first_max_and_bsums(orc):
    x = np.zeros(256, np.float32)
    # the first of the equal |x| is mx; it always gets code -127, so the sign
    # of d = 1 / (-127 / mx) tells which element came first
    x[10], x[200] = -2.0, 2.0
    d, qs, bs = _q8k_fields(orc.quantize_q8_K(x))
    assert qs[10] == -127 and qs[200] == 127 and d == np.float32(1) / (np.float32(-127) / np.float32(-2.0))
    x[10], x[200] = 2.0, -2.0
    d, qs, bs = _q8k_fields(orc.quantize_q8_K(x))
    assert qs[10] == -127 and qs[200] == 127 and d == np.float32(1) / (np.float32(-127) / np.float32(2.0))
    g = np.random.default_rng(7)
    x = g.standard_normal(1024).astype(np.float32)
    for i in range(4):
        d, qs, bs = _q8k_fields(orc.quantize_q8_K(x)[292 * i:292 * (i + 1)])
        assert np.array_equal(bs, qs.astype(np.int32).reshape(16, 16).sum(1))
        assert np.max(np.abs(qs.astype(np.int32))) == 127 and np.min(qs) >= -127
        xb = x[256 * i:256 * (i + 1)]
        assert np.max(np.abs(xb - qs * d)) <= abs(d) * 0.5 * (1 + 1e-5)
    z = orc.quantize_q8_K(np.zeros(512, np.float32))
    assert not z.any()


def q8k_tie_block():
    """A q8_K block whose first max-|x| element is -127, so iscale = -127 / -127 = 1 exactly
    and every other element n + 1/2 (n in [-100, 99]) lands on an exact tie; with the codes
    round-half-even gives: n when n is even, n + 1 when n is odd (half away from zero would
    give n + 1 for n >= 0 and n for n < 0)."""
    n = (np.arange(255) % 200) - 100
    x = np.concatenate([[-127.0], n + 0.5]).astype(np.float32)
    want = np.concatenate([[-127], np.where(n % 2 == 0, n, n + 1)]).astype(np.int8)
    return x, want


def test_q8_K_exact_ties_round_half_even(orc):
    x, want = q8k_tie_block()
    d, qs, bs = _q8k_fields(orc.quantize_q8_K(x))
    assert d == np.float32(1.0)
    assert np.array_equal(qs, want)
    assert np.array_equal(bs, want.astype(np.int32).reshape(16, 16).sum(1))


# ---------------------------------------------------------------- dots
def _deq_q8(qtype, xq, k):
    """dequantized activations (q * d) in fp64 from the block bytes"""
    if O.TYPES[qtype][2] == O.Q8_0:
        b = xq.reshape(-1, 34)
        return (b[:, 2:].view(np.int8).astype(np.float64) * b[:, :2].copy().view(np.float16).astype(np.float64)).ravel()
    b = xq.reshape(-1, 292)
    return (b[:, 4:260].view(np.int8).astype(np.float64) * b[:, 0:4].copy().view(np.float32).astype(np.float64)).ravel()


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K, O.IQ4_NL, O.IQ4_XS])
@pytest.mark.parametrize("k", [256, 512, 2048])
def test_vec_dot_textbook_identity(orc, qtype, k):
    from arcint_amd import synth
    rows = 16
    w = synth.weights(qtype, rows, k, seed=11 + qtype)
    x = synth.activations(1, k, seed=12).ravel()
    xq = orc.quantize_act(qtype, x)
    xd = _deq_q8(qtype, xq, k)
    rb = synth.row_bytes(qtype, k)
    for r in range(rows):
        wr = w[r * rb:(r + 1) * rb]
        wd = orc.dequantize(qtype, wr, k).astype(np.float64)
        terms = wd * xd
        exact = terms.sum()
        got = orc.vec_dot(qtype, k, wr, xq)
        # only the fp32 combine rounds: bounded by a few ulps of sum |terms|
        assert abs(got - exact) <= 1e-5 * np.abs(terms).sum() + 1e-30, (r, got, exact)


def test_mul_mat_threads_and_rows(orc):
    from arcint_amd import synth
    M, K, N = 37, 512, 3
    for qtype in (O.Q4_0, O.Q4_K):
        w = synth.weights(qtype, M, K, seed=2)
        x = synth.activations(N, K, seed=3)
        a = orc.mul_mat(qtype, w, M, K, x, threads=1)
        b = orc.mul_mat(qtype, w, M, K, x, threads=5)
        assert np.array_equal(a, b)
        rb = synth.row_bytes(qtype, K)
        for n in range(N):
            xq = orc.quantize_act(qtype, x[n])
            for m in (0, 17, M - 1):
                assert a[n, m] == orc.vec_dot(qtype, K, w[m * rb:(m + 1) * rb], xq)


def test_mul_mat_id_semantics(orc):
    from arcint_amd import synth
    M, K, E, T, n_used = 8, 256, 4, 3, 2
    qtype = O.Q4_K
    w = synth.weights(qtype, E * M, K, seed=4)
    ids = np.array([[0, 3], [2, -1], [1, 1]], np.int32)
    eb = synth.row_bytes(qtype, K) * M
    for ne11 in (1, n_used):
        x = synth.activations(T * ne11, K, seed=5).reshape(T, ne11, K)
        out = orc.mul_mat_id(qtype, w, M, K, E, x, ids)
        for t in range(T):
            for i in range(n_used):
                e = ids[t, i]
                if e < 0:
                    assert not out[t, i].any()
                    continue
                ref = orc.mul_mat(qtype, w[e * eb:(e + 1) * eb], M, K, x[t, i % ne11][None])[0]
                assert np.array_equal(out[t, i], ref)
