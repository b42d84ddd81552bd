"""The device weight image (host side, CPU only).

* pack/unpack round trips for every type, ragged row counts, partial 256-weight
  groups (Q4_0/Q8_0) and several matrices;
* the placement of every GGUF byte, checked against an independent statement
  of the layout (tile of 64 rows, group of 256 weights, 1 KB chunk planes);
* a numpy emulation of the GEMV kernel's per-chunk arithmetic on the packed
  image (which nibble meets which activation code, where each scale comes
  from), compared with the CPU oracle's ggml-cpu dot products;
* the GEMV launch plan: the waves cover the K axis, no work-group is left
  without groups, and the LDS of the cross-wave sum is what the plan says;
* the IQ4 codebook lookup's byte arithmetic (three v_perm_b32 per four codes,
  emulated) against the oracle's codebook for every byte value.
"""
import os

import numpy as np
import pytest

from arcint_amd import qmm, synth
from conftest import rel_err

TYPES = [qmm.Q4_0, qmm.Q8_0, qmm.Q4_K, qmm.Q5_K, qmm.Q6_K, qmm.IQ4_NL, qmm.IQ4_XS]
# type -> (chunk planes, tail bytes per row)
PLANES = {qmm.Q4_0: (9, 0), qmm.Q8_0: (17, 0), qmm.Q4_K: (9, 0), qmm.Q5_K: (11, 0), qmm.Q6_K: (13, 2),
          qmm.IQ4_NL: (9, 0), qmm.IQ4_XS: (8, 8)}
KV = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int64)


def shapes(qtype):
    blck, _ = synth.BLOCK[qtype]
    out = [(256 * 2, 64, 1), (256 * 3, 130, 1), (512, 7, 3), (1024, 64, 2)]
    if blck == 32:
        out += [(32 * 11, 65, 1), (32 * 9, 3, 2)]          # partial last group
    return out


def tg_bytes(qtype):
    nch, tail = PLANES[qtype]
    return nch * 1024 + 64 * tail


@pytest.mark.parametrize("qtype", TYPES)
def test_pack_unpack_roundtrip(qtype):
    for K, M, E in shapes(qtype):
        raw = synth.weights(qtype, M * E, K, seed=K + M)
        img = qmm.pack(qtype, (K, M, E), raw)
        assert img.nbytes == qmm.alloc_size(qtype, (K, M, E))
        assert img.nbytes % 256 == 0
        assert np.array_equal(qmm.unpack(qtype, (K, M, E), img), raw)


def expected_pieces(qtype, p):
    """(src offset in the block, size, chunk, byte in the chunk row, tail?) for block slot p"""
    if qtype in (qmm.Q4_0, qmm.IQ4_NL):
        return [(2, 16, p, 0, False), (0, 2, 8, 2 * p, False)]
    if qtype == qmm.Q8_0:
        return [(2, 16, 2 * p, 0, False), (18, 16, 2 * p + 1, 0, False), (0, 2, 16, 2 * p, False)]
    if qtype == qmm.Q4_K:
        return [(16 + 16 * c, 16, c, 0, False) for c in range(8)] + [(0, 16, 8, 0, False)]
    if qtype == qmm.Q5_K:   # d, dmin, scales[12] | qh[32] | qs[128]
        return ([(48 + 16 * c, 16, c, 0, False) for c in range(8)] + [(0, 16, 8, 0, False)]
                + [(16, 16, 9, 0, False), (32, 16, 10, 0, False)])
    if qtype == qmm.Q6_K:
        return ([(16 * c, 16, c, 0, False) for c in range(8)] + [(128 + 16 * c, 16, 8 + c, 0, False) for c in range(4)]
                + [(192, 16, 12, 0, False), (208, 2, None, 0, True)])
    return [(8 + 16 * c, 16, c, 0, False) for c in range(8)] + [(0, 8, None, 0, True)]


@pytest.mark.parametrize("qtype", TYPES)
def test_pack_placement(qtype):
    blck, bb = synth.BLOCK[qtype]
    bpg = 256 // blck
    nch, tail = PLANES[qtype]
    tg = tg_bytes(qtype)
    for K, M, E in shapes(qtype):
        raw = synth.weights(qtype, M * E, K, seed=7 + K).reshape(E, M, K // blck, bb)
        img = qmm.pack(qtype, (K, M, E), raw.ravel())
        G, nt = -(-K // 256), -(-M // 64)
        g = np.random.default_rng(K + M)
        for _ in range(200):
            e, m, kb = int(g.integers(E)), int(g.integers(M)), int(g.integers(K // blck))
            t, r, grp, p = m // 64, m % 64, kb // bpg, kb % bpg
            base = ((e * nt + t) * G + grp) * tg
            for src, size, chunk, off, is_tail in expected_pieces(qtype, p):
                at = base + (nch * 1024 + r * tail if is_tail else chunk * 1024 + r * 16 + off)
                assert np.array_equal(img[at:at + size], raw[e, m, kb, src:src + size]), (e, m, kb, src)
        # padding rows and padding blocks are zero
        used = np.zeros(img.nbytes, bool)
        for e in range(E):
            for m in range(M):
                t, r = m // 64, m % 64
                for kb in range(K // blck):
                    grp, p = kb // bpg, kb % bpg
                    base = ((e * nt + t) * G + grp) * tg
                    for src, size, chunk, off, is_tail in expected_pieces(qtype, p):
                        at = base + (nch * 1024 + r * tail if is_tail else chunk * 1024 + r * 16 + off)
                        used[at:at + size] = True
        assert not img[~used].any()
        assert used.sum() == raw.size


# ---------------------------------------------------------------- kernel arithmetic on the image
def image_planes(qtype, img, K, M):
    """chunks [M, G, nchunk, 16] and tail [M, G, tail] of a single matrix"""
    nch, tail = PLANES[qtype]
    tg = tg_bytes(qtype)
    G, nt = -(-K // 256), -(-M // 64)
    a = img[:nt * G * tg].reshape(nt, G, tg)
    ch = a[:, :, :nch * 1024].reshape(nt, G, nch, 64, 16).transpose(0, 3, 1, 2, 4).reshape(nt * 64, G, nch, 16)[:M]
    tl = None
    if tail:
        tl = a[:, :, nch * 1024:nch * 1024 + 64 * tail].reshape(nt, G, 64, tail).transpose(0, 2, 1, 3)
        tl = tl.reshape(nt * 64, G, tail)[:M]
    return ch.astype(np.int64), tl


def f16(lo, hi):
    return (lo.astype(np.uint16) | (hi.astype(np.uint16) << 8)).view(np.float16).astype(np.float32)


def q8_parts(orc, qtype, x):
    """codes [K], d per block, sums per (16 or 32) from the oracle's quantizer"""
    K = x.size
    q = orc.quantize_act(qtype, x)
    if orc.TYPES[qtype][2] == orc.Q8_0:
        b = q.reshape(K // 32, 34)
        return b[:, 2:].view(np.int8).astype(np.int64).ravel(), f16(b[:, 0], b[:, 1]), None
    b = q.reshape(K // 256, 292)
    d = b[:, :4].copy().view(np.float32).ravel()
    codes = b[:, 4:260].copy().view(np.int8).astype(np.int64).ravel()
    bsums = b[:, 260:].copy().view(np.int16).astype(np.int64).ravel()
    return codes, d, bsums


def emulate_gemv(qtype, img, K, M, codes, xd, bsums):
    ch, tl = image_planes(qtype, img, K, M)
    G = ch.shape[1]
    Kp = G * 256
    xc = np.zeros(Kp, np.int64)
    xc[:K] = codes
    xg = xc.reshape(G, 256)
    acc = np.zeros(M, np.float64)
    lo, hi = ch & 15, ch >> 4
    if qtype in (qmm.Q4_0, qmm.Q8_0, qmm.IQ4_NL):
        nb = K // 32
        xdp = np.zeros(G * 8, np.float32)
        xdp[:nb] = xd
        xdp = xdp.reshape(G, 8)
        for p in range(8):
            dw = f16(ch[:, :, 16 if qtype == qmm.Q8_0 else 8, 2 * p], ch[:, :, 16 if qtype == qmm.Q8_0 else 8, 2 * p + 1])
            xa, xb = xg[:, 32 * p:32 * p + 16], xg[:, 32 * p + 16:32 * p + 32]
            if qtype == qmm.Q4_0:
                s = (lo[:, :, p] * xa).sum(-1) + (hi[:, :, p] * xb).sum(-1) - 8 * (xa.sum(-1) + xb.sum(-1))
            elif qtype == qmm.IQ4_NL:
                s = (KV[lo[:, :, p]] * xa).sum(-1) + (KV[hi[:, :, p]] * xb).sum(-1)
            else:
                w0 = ch[:, :, 2 * p].astype(np.uint8).view(np.int8).astype(np.int64)
                w1 = ch[:, :, 2 * p + 1].astype(np.uint8).view(np.int8).astype(np.int64)
                s = (w0 * xa).sum(-1) + (w1 * xb).sum(-1)
            acc += (s * (dw * xdp[:, p])).sum(-1)
        return acc
    bs = bsums.reshape(G, 16)
    if qtype in (qmm.Q4_K, qmm.Q5_K):
        if qtype == qmm.Q5_K:   # fifth bits: byte 16 (c % 2) + i of qh, bit 2 (c // 2) (low) / + 1 (high)
            for c in range(8):
                qh = ch[:, :, 9 + (c & 1)]
                lo[:, :, c] |= ((qh >> (2 * (c // 2))) & 1) << 4
                hi[:, :, c] |= ((qh >> (2 * (c // 2) + 1)) & 1) << 4
        h = ch[:, :, 8].astype(np.uint8)
        d, dmin = f16(h[..., 0], h[..., 1]), f16(h[..., 2], h[..., 3])
        w = h.view(np.uint32).astype(np.uint64)             # [M, G, 4] dwords
        sc03, mn03 = w[..., 1] & 0x3f3f3f3f, w[..., 2] & 0x3f3f3f3f
        sc47 = (w[..., 3] & 0x0f0f0f0f) | ((w[..., 1] >> 2) & 0x30303030)
        mn47 = ((w[..., 3] >> 4) & 0x0f0f0f0f) | ((w[..., 2] >> 2) & 0x30303030)
        sc = [((sc03 >> (8 * i)) & 255) for i in range(4)] + [((sc47 >> (8 * i)) & 255) for i in range(4)]
        mn = [((mn03 >> (8 * i)) & 255) for i in range(4)] + [((mn47 >> (8 * i)) & 255) for i in range(4)]
        isc = np.zeros(d.shape, np.int64)
        for c in range(8):
            jl, xo = 2 * (c // 2), 64 * (c // 2) + 16 * (c % 2)
            sl = (lo[:, :, c] * xg[:, xo:xo + 16]).sum(-1)
            sh = (hi[:, :, c] * xg[:, xo + 32:xo + 48]).sum(-1)
            isc += sc[jl].astype(np.int64) * sl + sc[jl + 1].astype(np.int64) * sh
        imn = sum(mn[i].astype(np.int64) * (bs[:, 2 * i] + bs[:, 2 * i + 1]) for i in range(8))
        return (xd * (d * isc - dmin * imn)).sum(-1)
    if qtype == qmm.Q6_K:
        d = f16(tl[..., 0], tl[..., 1])
        scs = ch[:, :, 12].astype(np.uint8).view(np.int8).astype(np.int64)
        isum = np.zeros(d.shape, np.int64)
        for n in range(2):
            for lh in range(2):
                qh = ch[:, :, 8 + 2 * n + lh]
                for g in range(4):
                    ql = ch[:, :, 4 * n + 2 * (g & 1) + lh]
                    code = ((ql >> (0 if g < 2 else 4)) & 15) | (((qh >> (2 * g)) & 3) << 4)
                    is_ = 8 * n + 2 * g + lh
                    xo = 128 * n + 32 * g + 16 * lh
                    s = (code * xg[:, xo:xo + 16]).sum(-1) - 32 * bs[:, is_]
                    isum += scs[:, :, is_] * s
        return ((d * xd) * isum).sum(-1)
    # IQ4_XS
    kv = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int64)
    dw = f16(tl[..., 0], tl[..., 1])
    tl = tl.astype(np.int64)
    shi = tl[..., 2] | (tl[..., 3] << 8)
    slo = tl[..., 4] | (tl[..., 5] << 8) | (tl[..., 6] << 16) | (tl[..., 7] << 24)
    isum = np.zeros(dw.shape, np.int64)
    for ib in range(8):
        ls = ((slo >> (4 * ib)) & 15) | (((shi >> (2 * ib)) & 3) << 4)
        s = (kv[lo[:, :, ib]] * xg[:, 32 * ib:32 * ib + 16]).sum(-1) + (kv[hi[:, :, ib]] * xg[:, 32 * ib + 16:32 * ib + 32]).sum(-1)
        isum += (ls - 32) * s
    return ((dw * xd) * isum).sum(-1)


@pytest.mark.parametrize("qtype", TYPES)
def test_gemv_arithmetic_on_image(orc, qtype):
    blck, _ = synth.BLOCK[qtype]
    for K, M in [(1024, 70), (512, 64)] + ([(32 * 13, 65)] if blck == 32 else []):
        raw = synth.weights(qtype, M, K, seed=3 + K)
        x = synth.activations(1, K, seed=4 + K)
        img = qmm.pack(qtype, (K, M), raw)
        codes, xd, bsums = q8_parts(orc, qtype, x[0])
        got = emulate_gemv(qtype, img, K, M, codes, xd, bsums)
        ref = orc.mul_mat(qtype, raw, M, K, x)[0]
        assert rel_err(got, ref) <= 1e-5, qtype


# ---------------------------------------------------------------- launch plan
PLAN_SHAPES = [
    (qmm.Q4_K, 5120, 17408, 1), (qmm.Q4_K, 5120, 17408, 4), (qmm.Q6_K, 17408, 5120, 1), (qmm.Q6_K, 5120, 151936, 1),
    (qmm.Q4_0, 4096, 4096, 1), (qmm.Q4_0, 11008, 4096, 8), (qmm.Q8_0, 4096, 14336, 8), (qmm.IQ4_XS, 14336, 4096, 2),
    (qmm.Q4_0, 352, 65, 3), (qmm.Q4_K, 256, 1, 1), (qmm.Q8_0, 32, 5, 8), (qmm.IQ4_XS, 512, 2048, 5),
    (qmm.Q5_K, 5120, 17408, 1), (qmm.Q5_K, 4096, 4096, 6), (qmm.IQ4_NL, 640, 4096, 1), (qmm.IQ4_NL, 4096, 14336, 8),
    # wide MFMA tasks: 9..32 columns per weight pass, more in even passes (past 32, shapes the
    # GEMM does not take: few rows or few weight bytes)
    (qmm.Q4_K, 5120, 17408, 16), (qmm.Q4_K, 5120, 2048, 100), (qmm.Q4_0, 4096, 11008, 32), (qmm.Q8_0, 4096, 14336, 24),
    (qmm.IQ4_XS, 14336, 4096, 40), (qmm.IQ4_NL, 4096, 4096, 9), (qmm.Q6_K, 17408, 5120, 12), (qmm.Q5_K, 5120, 4096, 9),
]


@pytest.mark.parametrize("qtype,K,M,N", PLAN_SHAPES)
def test_gemv_plan(qtype, K, M, N):
    fake = qmm.Buffer(ptr=0x1000, size=1 << 44)
    info = qmm.describe_mul_mat(qmm.Tensor(fake, qtype, (K, M)), qmm.Tensor(fake, qmm.F32, (K, N)),
                                qmm.Tensor(fake, qmm.F32, (M, N)))
    # the MFMA kernel takes 3 and more columns of the types whose blocks it decodes, up to 32 a
    # weight pass; v_dot4 8; the columns spread evenly over the fewest passes
    mma = N >= 3 and qtype in (qmm.Q4_0, qmm.Q8_0, qmm.Q4_K, qmm.IQ4_XS, qmm.IQ4_NL, qmm.Q6_K)
    G, nt = -(-K // 256), -(-M // 64)
    if info["path"] == "gemv-fq":
        # the fused-quantization kernel: 1-2 columns, work-groups of up to 16 waves per 64-row
        # tile and task; K split among the waves and, for one column of any type but Q6_K or
        # a small image (at most 16 MiB), over KS work-groups of 4 waves (8 for Q8_0) with one
        # group each
        # (the K-slice tree); LDS holds each wave's quantized groups (320 B per group and
        # column), then the waves' sums
        W, spw, nc, KS = info["k_waves"], info["groups_per_wave"], info["cols_per_task"], info["k_slices"]
        # (3-16 columns as 2-column tasks on small products: at most 8 groups, 512 tile-groups)
        assert nc == min(N, 2) and info["tasks"] == -(-N // 2) and N <= 16
        if N > 2:
            assert G <= 8 and info["tasks"] * nt * G <= 512 and KS == 1
        assert 1 <= W <= 16 and KS * W * spw >= G and (KS - 1) * W * spw < G
        if KS == 1:
            assert (W - 1) * spw < G
        else:
            image = nt * G * {qmm.Q4_0: 18, qmm.Q8_0: 34, qmm.Q4_K: 144, qmm.Q5_K: 176, qmm.Q6_K: 210,
                              qmm.IQ4_XS: 136, qmm.IQ4_NL: 18}[qtype] * (8 if qtype in (qmm.Q4_0, qmm.Q8_0, qmm.IQ4_NL) else 1) * 64
            assert N == 1 or (N == 2 and qtype == qmm.Q8_0) or image <= 16 << 20
            assert W == (8 if qtype == qmm.Q8_0 else 4) and spw == 1
        assert info["workgroups"] == info["tasks"] * nt * KS and info["threads"] == 64 * W
        assert info["lds_bytes"] == max(W * spw * nc * 320, W * 2 * nc * 64 * 4)
        return
    assert info["path"] == ("gemv-mfma" if mma else "gemv")
    W, KS, spw, nc = info["k_waves"], info["k_slices"], info["groups_per_wave"], info["cols_per_task"]
    cap = 32 if mma else 8
    assert nc == -(-N // -(-N // cap))
    assert 1 <= W <= 8 and KS >= 1 and spw >= 1
    assert KS * W * spw >= G                             # the waves cover K
    assert (KS - 1) * W * spw < G                        # no work-group without groups
    assert info["tasks"] == -(-N // nc)
    tw = info["tiles_per_wg"]
    assert info["threads"] == 64 * W * tw
    assert info["workgroups"] == info["tasks"] * -(-nt // tw) * KS
    if mma:
        # TW tiles x W waves splitting K; the K range's activations are staged in LDS: 256 zero
        # bytes, then per column and group the codes (272 B), Q4_K split sums (16 B) and the
        # scales (4 B per block); the W waves' sums reuse it
        # (cm = the kernel's columns: 8, 16 or 32; the LDS holds 24 x 8 / cm groups)
        cm = 8 if nc <= 8 else 16 if nc <= 16 else 32
        assert 1 <= tw <= 4 and W * tw <= 4 and W * spw <= 24 * 8 // cm
        nsb = 8 if qtype in (qmm.Q4_0, qmm.Q8_0, qmm.IQ4_NL) else 1
        stage = 256 + W * spw * cm * (272 + (16 if qtype == qmm.Q4_K else 0) + 4 * nsb)
        assert info["lds_bytes"] == max(stage, W * tw * cm * 64 * 4 if W > 1 else 0)
    else:
        assert tw == 1
        assert info["lds_bytes"] == (W * nc * 64 * 4 if W > 1 else 0)


# the streaming GEMM of the block types (one float scale per 32 weights) has Q4_K's frame (the
# plan rule below: test_gemm_stream_q4k_plan), without the candidate of two row-half waves per
# K slice, whose stages are shared by too few waves
GEMM3_SHAPES = [(qmm.Q4_0, 4096, 4096, 512), (qmm.Q4_0, 11008, 4096, 512), (qmm.Q4_0, 4096, 11008, 512),
                (qmm.Q8_0, 4096, 14336, 64), (qmm.IQ4_NL, 800, 130, 33), (qmm.Q4_0, 4096, 4096, 100)]


@pytest.mark.parametrize("qtype,K,M,N", GEMM3_SHAPES)
def test_gemm_stream_plan(qtype, K, M, N, monkeypatch):
    monkeypatch.setenv("QMM_GEMM_MIN_COLS", "16")                 # (small shapes: the GEMM regardless)
    fake = qmm.Buffer(ptr=0x1000, size=1 << 44)
    info = qmm.describe_mul_mat(qmm.Tensor(fake, qtype, (K, M)), qmm.Tensor(fake, qmm.F32, (K, N)),
                                qmm.Tensor(fake, qmm.F32, (M, N)))
    assert info["path"] == "gemm-stream"
    check_kq_plan(info, -(-K // 256), M, N, [c for c in KQ_CANDS if c[0] != 2])


# Q4_K on the streaming GEMM: a wave per (32-row half of a tile, pair of 32-column tiles, K
# slice); U row-half waves per K slice share the staged activations, KS slices per work-group.
# (U, KS) minimizes rounds of work-groups on 256 CUs (12-wave groups: one per CU, whole rounds;
# 4-wave: three per CU, a partial last round counted as its fraction) times super-blocks per
# slice, ties to the earlier candidate; LDS: two 18 KB stages per slice (+ a 1 KB slot when 18
# units do not divide over U), or the slices' sums if larger
# past the column crossover the GEMM is taken when its launch gives every SIMD a wave (row units x
# column units x K slices >= 1024), else the GEMV's split-K tasks
@pytest.mark.parametrize("qtype,K,M,N,path", [(qmm.Q4_K, 2048, 512, 256, "gemv-mfma"), (qmm.Q4_K, 5120, 17408, 512, "gemm-stream"),
                                              (qmm.Q4_K, 5120, 1024, 512, "gemm-stream"), (qmm.Q4_0, 4096, 4096, 64, "gemv-mfma"),
                                              (qmm.Q4_0, 4096, 4096, 128, "gemm-stream"),
                                              (qmm.Q4_0, 4096, 4096, 512, "gemm-stream"), (qmm.Q6_K, 17408, 5120, 512, "gemm-stream"),
                                              # fewer than 1024 waves: the GEMM when the GEMV's passes stream >= 90 MB
                                              # (Q6_K 400 MB), measured crossovers
                                              (qmm.Q4_K, 5120, 17408, 40, "gemm-stream"), (qmm.Q4_K, 5120, 12288, 48, "gemm-stream"),
                                              (qmm.Q4_K, 6144, 5120, 64, "gemv-mfma"), (qmm.Q4_K, 5120, 17408, 32, "gemv-mfma"),
                                              (qmm.Q6_K, 17408, 5120, 128, "gemv-mfma"), (qmm.Q6_K, 17408, 5120, 192, "gemm-stream"),
                                              (qmm.Q6_K, 5120, 151936, 64, "gemm-stream"), (qmm.IQ4_XS, 14336, 4096, 48, "gemv-mfma"),
                                              (qmm.Q5_K, 5120, 17408, 16, "gemm-stream")])
def test_gemm_fill_rule(qtype, K, M, N, path):
    fake = qmm.Buffer(ptr=0x1000, size=1 << 44)
    info = qmm.describe_mul_mat(qmm.Tensor(fake, qtype, (K, M)), qmm.Tensor(fake, qmm.F32, (K, N)),
                                qmm.Tensor(fake, qmm.F32, (M, N)))
    assert info["path"] == path


KQ_CANDS = [(12, 1, 1), (6, 2, 1), (4, 3, 1), (3, 4, 1), (4, 1, 3), (2, 2, 3)]
GEMM3_KQ_SHAPES = [(5120, 17408, 512), (5120, 12288, 512), (5120, 1024, 512), (6144, 5120, 512),
                   (4096, 4096, 128), (256, 130, 33), (17408, 5120, 512), (5120, 151936, 512)]


def kq_tail(nwg, U, KS, G):
    """the blocks of a one-slice launch past a whole number per CU (nwg % 256) in K pieces:
    (whole blocks, pieces per tail block); ts in 2..4 minimizes the load per CU
    ceil(tail ts / 256) / ts below 1, at least two stages a piece and the last piece not empty,
    ties to fewer pieces"""
    if KS != 1:
        return nwg, 1
    full = nwg // 256 * 256
    rest = nwg - full
    best = (1, 1)                                                 # load per CU: num / den
    for ts in range(2, 5):
        pk = -(-G // ts)
        if rest == 0 or rest > 256 or pk < 2 or (ts - 1) * pk >= G:
            continue
        r = -(-(rest * ts) // 256)
        if r * best[1] < best[0] * ts:
            best = (r, ts)
    return (full, best[1]) if best[1] > 1 else (nwg, 1)


def check_kq_plan(info, G, M, N, cands):
    """the streaming GEMMs' launch plan: (U, KS) minimizes rounds of work-groups on 256 CUs (12-wave
    groups: one per CU, whole rounds; 4-wave: three per CU, a partial last round counted as its
    fraction) times groups per slice, U = 2 paying 1/16 more (its stage shared by two waves), ties
    to the earlier candidate; a one-slice launch runs its blocks past a whole number per CU in K pieces
    (kq_tail)"""
    nrh, ncp = 2 * -(-M // 64), -(-(-(-N // 32)) // 2)
    best = None
    for U, ks, per_cu in cands:
        sps = -(-G // ks)
        mbn = -(-nrh // U)
        slots = 256 * per_cu
        nwg = mbn * ncp
        rounds = max(64, -(-(nwg * 64) // slots)) if per_cu > 1 else 64 * -(-nwg // slots)
        cost = rounds * sps * 17 // 16 if U == 2 else rounds * sps     # (dense: two waves share a stage)
        if best is None or cost < best[0]:
            best = (cost, U, -(-G // sps), sps, mbn)
    _, U, KS, sps, mbn = best
    assert info["k_slices"] == KS and info["cols_per_task"] == 64
    assert info["threads"] == 64 * U * KS
    full, ts = kq_tail(mbn * ncp, U, KS, G)
    assert info["workgroups"] == 8 * -(-full // 8) + 8 * -(-((mbn * ncp - full) * ts) // 8)
    assert info["groups_per_wave"] == sps
    lds = max(KS * 2 * 18 * 1024 + (1024 if 18 % U else 0), (KS - 1) * U * 32 * 64 * 4)
    assert info["lds_bytes"] == lds <= 160 * 1024


@pytest.mark.parametrize("qtype", [qmm.Q4_K, qmm.Q6_K, qmm.Q5_K, qmm.IQ4_XS])
@pytest.mark.parametrize("K,M,N", GEMM3_KQ_SHAPES)
def test_gemm_stream_kquant_plan(qtype, K, M, N):
    fake = qmm.Buffer(ptr=0x1000, size=1 << 44)
    os.environ["QMM_GEMM_MIN_COLS"] = "16"
    try:
        info = qmm.describe_mul_mat(qmm.Tensor(fake, qtype, (K, M)), qmm.Tensor(fake, qmm.F32, (K, N)),
                                    qmm.Tensor(fake, qmm.F32, (M, N)))
    finally:
        del os.environ["QMM_GEMM_MIN_COLS"]
    assert info["path"] == "gemm-stream"
    check_kq_plan(info, K // 256, M, N, KQ_CANDS)


# IQ4_NL 14336 x 4096 x 512: 896 blocks of 4 row-half waves = 3 x 256 + 128; the 768 run whole,
# the other 128 as two K halves each (1024 work-groups); QMM_GEMM3_TAIL=0: whole blocks.  Q4_K
# 17408 x 5120 x 512: 1088 blocks = 4 x 256 + 64, the 64 as four K pieces each (1280).
@pytest.mark.parametrize("qtype,K,M,tail,wgs", [(qmm.IQ4_NL, 4096, 14336, "1", 768 + 2 * 128),
                                                (qmm.IQ4_NL, 4096, 14336, "0", 896),
                                                (qmm.Q4_K, 5120, 17408, "1", 1024 + 4 * 64),
                                                (qmm.Q4_K, 5120, 17408, "0", 1088)])
def test_gemm_tail_split_plan(qtype, K, M, tail, wgs, monkeypatch):
    monkeypatch.setenv("QMM_GEMM3_TAIL", tail)
    fake = qmm.Buffer(ptr=0x1000, size=1 << 44)
    info = qmm.describe_mul_mat(qmm.Tensor(fake, qtype, (K, M)), qmm.Tensor(fake, qmm.F32, (K, 512)),
                                qmm.Tensor(fake, qmm.F32, (M, 512)))
    assert info["path"] == "gemm-stream" and info["threads"] == 256 and info["k_slices"] == 1
    assert info["workgroups"] == wgs


# ---- the IQ4 codebook lookup's byte arithmetic (qmm_device.h: iq4_lookup, iq4_lookup8,
# iq4_lookup_r), on the CPU: v_perm_b32 emulated for selector bytes 0-7, every byte value in
# every position, against the oracle's codebook (ggml-quants.c kvalues_iq4nl)

def _perm(hi, lo, sel):
    """v_perm_b32 for selector bytes 0-7: byte i of the result is byte sel.i of {hi:lo}."""
    hi, lo, sel = np.broadcast_arrays(np.asarray(hi, np.uint32), np.asarray(lo, np.uint32), np.asarray(sel, np.uint32))
    both = (hi.astype(np.uint64) << np.uint64(32)) | lo.astype(np.uint64)
    out = np.zeros(lo.shape, np.uint64)
    for i in range(4):
        s = (sel >> np.uint32(8 * i)) & np.uint32(0xFF)
        assert int(s.max()) <= 7
        out |= ((both >> (np.uint64(8) * s.astype(np.uint64))) & np.uint64(0xFF)) << np.uint64(8 * i)
    return out.astype(np.uint32)


def _kv_words(kv):
    b = (np.asarray(kv, np.int64) & 0xFF).astype(np.uint32)
    return [np.uint32(b[4 * i] | (b[4 * i + 1] << 8) | (b[4 * i + 2] << 16) | (b[4 * i + 3] << 24))
            for i in range(4)]


def _lookup_r(x, k):
    """iq4_lookup_r: the codes in bits 0-3 of each byte of x, bits 4-7 ignored."""
    il = x & np.uint32(0x07070707)
    sl = ((x >> np.uint32(1)) & np.uint32(0x04040404)) | np.uint32(0x03020100)
    return _perm(_perm(k[3], k[2], il), _perm(k[1], k[0], il), sl)


def _lookup8(q, k):
    """iq4_lookup8: both nibbles of q's four bytes, the shift shared."""
    t = q >> np.uint32(4)
    il, ih = q & np.uint32(0x07070707), t & np.uint32(0x07070707)
    sl = ((q >> np.uint32(1)) & np.uint32(0x04040404)) | np.uint32(0x03020100)
    sh = ((t >> np.uint32(1)) & np.uint32(0x04040404)) | np.uint32(0x03020100)
    return (_perm(_perm(k[3], k[2], il), _perm(k[1], k[0], il), sl),
            _perm(_perm(k[3], k[2], ih), _perm(k[1], k[0], ih), sh))


def _codes(v, sh):
    return [(v >> np.uint32(8 * i + sh)) & np.uint32(0xF) for i in range(4)]


def _decoded(v):
    return [(v >> np.uint32(8 * i)) & np.uint32(0xFF) for i in range(4)]


def test_iq4_lookup_bytes(orc):
    kv = np.array(orc.kvalues(), np.int64)
    assert kv.tolist() == KV.tolist()
    k = _kv_words(kv)
    table = (kv & 0xFF).astype(np.uint32)
    rng = np.random.default_rng(7)
    b = np.arange(256, dtype=np.uint32)
    # every byte value in each of the four positions (the others random), then random dwords
    qs = [np.concatenate([b << np.uint32(8 * p) | (rng.integers(0, 2**32, 256, dtype=np.uint64).astype(np.uint32)
                                                  & ~np.uint32(0xFF << (8 * p)))
                          for p in range(4)]),
          rng.integers(0, 2**32, 4096, dtype=np.uint64).astype(np.uint32)]
    for q in qs:
        lo, hi = _lookup8(q, k)
        for got, sh in ((lo, 0), (hi, 4)):
            for g, c in zip(_decoded(got), _codes(q, sh)):
                assert np.array_equal(g, table[c])
        # the single-nibble form on an unmasked shift (the streaming GEMM's use)
        for sh in (0, 4):
            for g, c in zip(_decoded(_lookup_r(q >> np.uint32(sh), k)), _codes(q, sh)):
                assert np.array_equal(g, table[c])
